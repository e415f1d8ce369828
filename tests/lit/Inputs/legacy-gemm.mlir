module attributes {frisk.legacy_semantics = "tensor_v1", frisk.target = "gfx950"} {
  frisk.kernel @g(memref<64x32xf16, 1>, memref<32x64xf16, 1>, memref<64x64xf32, 1>) {
  ^bb0(%arg0: memref<64x32xf16, 1>, %arg1: memref<32x64xf16, 1>, %arg2: memref<64x64xf32, 1>):
    frisk.gemm(%arg0, %arg1, %arg2) {K = 32 : i64, M = 64 : i64, N = 64 : i64, clear_accum = true, frisk.legacy_semantics = "tensor_v1", policy = #frisk.gemm_warp_policy<Square>, transA = false, transB = false} : memref<64x32xf16, 1>, memref<32x64xf16, 1>, memref<64x64xf32, 1>
    frisk.end
  }
}
