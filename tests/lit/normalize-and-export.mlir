// RUN: frisk-opt %s --frisk-normalize-layout-ir -verify-each | FileCheck %s
// RUN: frisk-opt %s --frisk-normalize-layout-ir --frisk-infer-layouts -verify-each | FileCheck %s --check-prefix=LAYOUT
// RUN: frisk-opt %s --frisk-normalize-layout-ir --frisk-infer-layouts --frisk-export-execution | FileCheck %s --check-prefix=PACKET
// RUN: frisk-opt %s --frisk-normalize-layout-ir --frisk-infer-layouts --frisk-export-execution='output=%t.json minify' > %t.mlir
// RUN: FileCheck %s --check-prefix=LAYOUT < %t.mlir
// RUN: FileCheck %s --check-prefix=MINI < %t.json

// A legacy single-tile program (the builder's ops, as ffi/ir.cpp creates
// them): a GEMM accumulated into a zero-filled Local fragment, a row maximum
// merged into a -inf vector, both stored.  Normalization lowers them as
// lib/Dialect/Frisk/Transforms/LegacyFragmentNormalization.cpp does
// (gemm -> frisk.mma from a zero init, reduce -> frisk.reduce_tensor plus
// arith.maximumf with the old value, copies to Global -> tile_store).

// CHECK-LABEL: frisk.kernel @gemm_rowmax
// CHECK: %alloc = memref.alloc() : memref<64x32xf16, 3>
// CHECK: frisk.copy %{{.*}}[], %{{.*}}[] {dstExtents = array<i64: 64, 32>
// CHECK: %[[ZERO:.*]] = arith.constant dense<0.000000e+00> : tensor<64x64xf32>
// CHECK: %[[ACC:.*]] = frisk.mma %{{.*}}, %{{.*}}, %[[ZERO]] {frisk.execution_threads = 128 : i64, k = 32 : i64, m = 64 : i64, n = 64 : i64}
// CHECK: %[[NEGINF:.*]] = arith.constant dense<0xFF800000> : tensor<64xf32>
// CHECK: %[[MAX:.*]] = frisk.reduce_tensor %[[ACC]] {dim = 1 : i64, frisk.execution_threads = 128 : i64, kind = "max"}
// CHECK: %[[MERGED:.*]] = arith.maximumf %[[NEGINF]], %[[MAX]] : tensor<64xf32>
// CHECK: frisk.tile_store %[[ACC]], %{{.*}} : tensor<64x64xf32>, memref<64x64xf32, 1>
// CHECK: frisk.tile_store %[[MERGED]], %{{.*}} : tensor<64xf32>, memref<64xf32, 1>
// CHECK-NOT: frisk.gemm
// CHECK-NOT: frisk.reduce %

// LAYOUT: module attributes {{{.*}}frisk.layout_cost_model = "cdna4-layout-v1"
// LAYOUT: frisk.mma
// LAYOUT-SAME: form = "ss"
// The builder's GEMM carries policy Square, which fixes the wave grid (a
// non-Auto policy gives one geometry, SM90MmaLayoutProof.cpp:25-62): two
// waves over 64x64 as 1x2; the MFMA atom is the solver's choice.
// LAYOUT-SAME: atom = "v_mfma_f32_{{32x32x16|16x16x32}}_f16", wave_grid = [1, 2]
// LAYOUT-SAME: policy = "Square"
// LAYOUT: frisk.reduce_tensor
// LAYOUT-SAME: frisk.reduction_contract = #frisk.reduction_contract<

// PACKET: "schema_version": 1
// PACKET: "target": "gfx950"
// PACKET: "name": "frisk.reduce_tensor"
// PACKET-SAME: "fibers": [
// MINI: {"schema_version":1,"target":"gfx950",
module attributes {frisk.legacy_semantics = "tensor_v1", frisk.target = "gfx950"} {
  frisk.kernel @gemm_rowmax(memref<64x32xf16, 1>, memref<32x64xf16, 1>, memref<64x64xf32, 1>, memref<64xf32, 1>) {
  ^bb0(%arg0: memref<64x32xf16, 1>, %arg1: memref<32x64xf16, 1>, %arg2: memref<64x64xf32, 1>, %arg3: memref<64xf32, 1>):
    frisk.parallel (%arg4) = (1), threads = 128 {
      %0 = frisk.alloc_buffer {alignment = 0 : i64} -> memref<64x32xf16, 3>
      %1 = frisk.alloc_buffer {alignment = 0 : i64} -> memref<32x64xf16, 3>
      %2 = frisk.alloc_buffer {alignment = 0 : i64} -> memref<64x64xf32>
      %3 = frisk.alloc_buffer {alignment = 0 : i64} -> memref<64xf32>
      frisk.copy %arg0[], %0[] {dstExtents = array<i64: 64, 32>, srcExtents = array<i64: 64, 32>} : memref<64x32xf16, 1>, memref<64x32xf16, 3>
      frisk.copy %arg1[], %1[] {dstExtents = array<i64: 32, 64>, srcExtents = array<i64: 32, 64>} : memref<32x64xf16, 1>, memref<32x64xf16, 3>
      frisk.fill %2 {value = 0.000000e+00 : f32} : memref<64x64xf32>
      frisk.gemm(%0, %1, %2) {K = 32 : i64, M = 64 : i64, N = 64 : i64, clear_accum = false, frisk.legacy_semantics = "tensor_v1", policy = #frisk.gemm_warp_policy<Square>, transA = false, transB = false} : memref<64x32xf16, 3>, memref<32x64xf16, 3>, memref<64x64xf32>
      frisk.fill %3 {value = 0xFF800000 : f32} : memref<64xf32>
      frisk.reduce %2, %3 {clear = false, dim = 1 : i64, frisk.legacy_semantics = "tensor_v1", kind = "max"} : memref<64x64xf32>, memref<64xf32>
      frisk.copy %2[], %arg2[] {dstExtents = array<i64: 64, 64>, srcExtents = array<i64: 64, 64>} : memref<64x64xf32>, memref<64x64xf32, 1>
      frisk.copy %3[], %arg3[] {dstExtents = array<i64: 64>, srcExtents = array<i64: 64>} : memref<64xf32>, memref<64xf32, 1>
      frisk.end
    }
    frisk.end
  }
}