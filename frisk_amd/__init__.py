"""frisk_amd: MI355X-native GEMM and attention path of the Frisk tile compiler.

The package namespace is the reference's `import frisk as F` surface
(python/frisk/__init__.py:1-4): every name of the `frisk_ffi.ir` builder
module (context, builder, module, AffineMap, MemorySpace, the `frisk`
submodule with its op classes, ...) plus FriskHelper, create_context and
create_session.  On top of that:

execute  -- run a GEMM / attention tile program on the GPU (C-ABI)
execute_packet / plan_packet -- run an execution packet written by
            frisk.export_execution (after frisk.infer_layouts)
variants -- the compiled GEMM kernel variants and the MMA contracts they
            execute
parse_module -- read textual tile IR (the printed form, or MLIR's generic
            operation form) back into a module; `python -m frisk_amd.opt`
            is the frisk-opt-like driver over it
runtime  -- ctypes binding of libfrisk_hip.so (include/frisk_hip.h)
build    -- ahead-of-time build of libfrisk_hip.so (hipcc, gfx950) and of
            the frisk_ffi extension (g++, pybind11)

The builder names are resolved lazily, so `python -m frisk_amd.build` and
`frisk_amd.runtime` work before the extension is built.
"""
from __future__ import annotations

import sys as _sys

_IR = None


def _ir():
    """The `frisk_ffi.ir` module, loaded on first use."""
    global _IR
    if _IR is None:
        import importlib
        try:
            frisk_ffi = importlib.import_module(__name__ + ".frisk_ffi")
        except ImportError as e:  # pragma: no cover - build problem
            raise ImportError("frisk_amd.frisk_ffi is not built: run `python -m frisk_amd.build`") from e
        _IR = frisk_ffi.ir
        # Make `frisk_amd.frisk_ffi.ir` importable as a module path, like the
        # reference's `from .frisk_ffi.ir import *`.
        _sys.modules.setdefault(__name__ + ".frisk_ffi.ir", _IR)
        _sys.modules.setdefault(__name__ + ".frisk_ffi.ir.frisk", _IR.frisk)
    return _IR


_HELPERS = ("FriskHelper", "create_context", "create_session")


def parse_module(text: str, context=None):
    """Parse textual tile IR into a module (in `context`, or a new one that
    the module keeps alive as `module.context`)."""
    from .common import utils
    ctx = context if context is not None else utils.create_context()
    module = _ir().frisk.parse_module(text, ctx)
    module.context = ctx
    return module


def __getattr__(name: str):
    if name in _HELPERS:
        from .common import utils
        return getattr(utils, name)
    if name == "execute":
        from .executor import execute
        return execute
    if name in ("execute_packet", "plan_packet"):
        from . import packet
        return getattr(packet, name)
    if name == "parse_module":
        return parse_module
    if name.startswith("__") or name == "frisk_ffi":
        raise AttributeError(name)
    ir = _ir()
    if hasattr(ir, name):
        return getattr(ir, name)
    raise AttributeError(f"module 'frisk_amd' has no attribute '{name}'")


def __dir__():
    names = set(globals()) | set(_HELPERS) | {"execute", "execute_packet", "plan_packet"}
    try:
        names |= {n for n in dir(_ir()) if not n.startswith("_")}
    except ImportError:
        pass
    return sorted(names)
