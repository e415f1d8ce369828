// RUN: not frisk-opt %s --frisk-infer-layouts 2>&1 | FileCheck %s --check-prefix=TARGET
// RUN: not frisk-opt %s --frisk-infer-layouts='beam-width=x' 2>&1 | FileCheck %s --check-prefix=VALUE
// RUN: not frisk-opt %s --frisk-infer-layouts='seed-beam-solution' 2>&1 | FileCheck %s --check-prefix=OPTION
// RUN: not frisk-opt %s --frisk-bogus 2>&1 | FileCheck %s --check-prefix=PASS
// RUN: not frisk-opt %S/Inputs/parse-error.mlir 2>&1 | FileCheck %s --check-prefix=PARSE
// RUN: not frisk-opt %S/Inputs/legacy-gemm.mlir --frisk-infer-layouts 2>&1 | FileCheck %s --check-prefix=ORDER
// RUN: not frisk-opt %S/Inputs/legacy-gemm.mlir --frisk-normalize-layout-ir='target=sm_90a' 2>&1 | FileCheck %s --check-prefix=NORM

// Diagnostics of the driver and its passes.  This module asks for the
// reference's SM90 target, which the CDNA4 layout target refuses.

// TARGET: error: --frisk-infer-layouts: layout-inference: cdna4-target: requires frisk.target = "gfx950"
// VALUE: error: option beam-width needs an integer (got 'x')
// OPTION: error: --frisk-infer-layouts: unknown option(s) seed-beam-solution
// PASS: frisk-opt: error: unknown option or pass '--frisk-bogus'
// PARSE: parse-error.mlir:4:16: error: use of undefined value %undefined
// ORDER: error: --frisk-infer-layouts: layout-inference: input-verification: run frisk.normalize_layout_ir first (frisk.gemm)
// NORM: error: --frisk-normalize-layout-ir: 'frisk.gemm' op cdna4-mma-target: explicit gfx950 target required



module attributes {frisk.target = "sm_90a"} {
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
