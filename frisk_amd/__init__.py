"""frisk_amd: MI355X-native GEMM and attention path of the Frisk tile compiler.

runtime  -- ctypes binding of libfrisk_hip.so (include/frisk_hip.h)
build    -- ahead-of-time hipcc build of that library for gfx950
"""
