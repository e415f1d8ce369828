// RUN: frisk-opt %s --frisk-infer-layouts='analysis-only dump-analysis' 2>&1 | FileCheck %s --check-prefix=GRAPH
// RUN: frisk-opt %s --frisk-infer-layouts -verify-each > %t.once
// RUN: FileCheck %s < %t.once
// RUN: frisk-opt %t.once --frisk-infer-layouts -verify-each > %t.twice
// RUN: diff %t.once %t.twice

// One MFMA product with both operands in LDS ("ss") and one with A in
// registers ("rs"), as in the reference's test/Transforms/infer-gemm-layout.mlir
// (there for sm_90a wgmma; here for gfx950 MFMA).

// GRAPH: frisk-infer-layouts analysis
// GRAPH: hard instruction-contract mma#0
// GRAPH: solution: solved method=exact

// CHECK-LABEL: frisk.kernel @ss
// CHECK: memref.alloc() {alignment = 1024 : i64, frisk.storage = #frisk.storage<space = "lds", row_bytes = 32, swizzle = "c ^ ((r >> 3) & 1)">}
// CHECK: frisk.mma
// CHECK-SAME: form = "ss"
// CHECK-SAME: frisk.execution_threads = 128 : i64
// CHECK-SAME: frisk.mma_contract = #frisk.mma_contract<{atom = "v_mfma_f32_32x32x16_f16", wave_grid = [1, 2]
// CHECK-LABEL: frisk.kernel @rs
// CHECK: frisk.mma
// CHECK-SAME: form = "rs"
// CHECK-SAME: atom = "v_mfma_f32_32x32x16_bf16"
module attributes {frisk.target = "gfx950"} {
  frisk.kernel @ss() {
    frisk.parallel (%i) = (1), threads = 128 {
      %a = memref.alloc() {alignment = 1024 : i64} : memref<64x16xf16, 3>
      %b = memref.alloc() {alignment = 1024 : i64} : memref<16x64xf16, 3>
      %av = frisk.layout_view %a : memref<64x16xf16, 3> -> memref<64x16xf16, 3>
      %bv = frisk.layout_view %b : memref<16x64xf16, 3> -> memref<16x64xf16, 3>
      %zero = arith.constant dense<0.0> : tensor<64x64xf32>
      %r = frisk.mma %av, %bv, %zero {k = 16 : i64, m = 64 : i64, n = 64 : i64} : memref<64x16xf16, 3>, memref<16x64xf16, 3>, tensor<64x64xf32> -> tensor<64x64xf32>
      frisk.end
    }
    frisk.end
  }
  frisk.kernel @rs() {
    frisk.parallel (%j) = (1), threads = 128 {
      %a = arith.constant dense<1.0> : tensor<64x16xbf16>
      %b = memref.alloc() {alignment = 1024 : i64} : memref<16x64xbf16, 3>
      %bv = frisk.layout_view %b : memref<16x64xbf16, 3> -> memref<16x64xbf16, 3>
      %zero = arith.constant dense<0.0> : tensor<64x64xf32>
      %r = frisk.mma %a, %bv, %zero {k = 16 : i64, m = 64 : i64, n = 64 : i64} : tensor<64x16xbf16>, memref<16x64xbf16, 3>, tensor<64x64xf32> -> tensor<64x64xf32>
      frisk.end
    }
    frisk.end
  }
}
