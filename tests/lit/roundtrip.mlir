// RUN: frisk-opt %s > %t.1
// RUN: frisk-opt %t.1 > %t.2
// RUN: diff %t.1 %t.2
// RUN: FileCheck %s < %t.1

// Every custom form of the tile IR prints back as it was read: the grid of
// a tiled reduction with affine tile offsets, frisk.for / frisk.block bodies
// (implicit terminators), scf.for with iter_args, generic-form ops, and the
// attribute kinds (typed integers and floats, hex floats, arrays, maps,
// dense splats, dialect attributes, strings).

// CHECK-LABEL: frisk.kernel @tiles
// CHECK: frisk.parallel (%[[I:.*]], %[[J:.*]]) = (4, 2), threads = 256 {
// CHECK: frisk.copy %arg0[%[[I]] * 64, %[[J]] * 128], %{{.*}}[]
// CHECK: frisk.for %{{.*}} = 0 to 128 step = 32 {
// CHECK: frisk.block (%{{.*}}, %{{.*}}) to (16, 8) {
// CHECK: scf.for %{{.*}} = %c0 to %c4 step %c1 iter_args(%{{.*}} = %cst) -> (tensor<16xf32>) {
// CHECK: "math.exp"(%{{.*}}) {note = "kept", scale = 1.250000e-01 : f32} : (tensor<16xf32>) -> (tensor<16xf32>)
// CHECK: scf.yield %{{.*}} : tensor<16xf32>
// CHECK: frisk.fill %{{.*}} {value = 0xFF800000 : f32} : memref<64x128xf32>
module attributes {frisk.target = "gfx950"} {
  frisk.kernel @tiles(memref<256x256xf32, 1>, memref<256x256xbf16, 1>) {
  ^bb0(%arg0: memref<256x256xf32, 1>, %arg1: memref<256x256xbf16, 1>):
    frisk.parallel (%arg2, %arg3) = (4, 2), threads = 256 {
      %0 = frisk.alloc_buffer {alignment = 16 : i64} -> memref<64x128xf32>
      %1 = frisk.alloc_buffer {alignment = 0 : i64} -> memref<64x128xbf16, 3>
      frisk.copy %arg0[%arg2 * 64, %arg3 * 128 + 0], %0[] {dstExtents = array<i64: 64, 128>, srcExtents = array<i64: 64, 128>} : memref<256x256xf32, 1>, memref<64x128xf32>
      frisk.for %arg4 = 0 to 128 step = 32 {
        frisk.block (%arg5, %arg6) to (16, 8) {
        }
      }
      %c0 = arith.constant 0 : index
      %c1 = arith.constant 1 : index
      %c4 = arith.constant 4 : index
      %cst = arith.constant dense<0.000000e+00> : tensor<16xf32>
      %2 = scf.for %arg7 = %c0 to %c4 step %c1 iter_args(%arg8 = %cst) -> (tensor<16xf32>) {
        %3 = "math.exp"(%arg8) {note = "kept", scale = 1.250000e-01 : f32} : (tensor<16xf32>) -> (tensor<16xf32>)
        scf.yield %3 : tensor<16xf32>
      }
      frisk.fill %0 {value = 0xFF800000 : f32} : memref<64x128xf32>
      frisk.copy %0[], %1[] {dstExtents = array<i64: 64, 128>, srcExtents = array<i64: 64, 128>} : memref<64x128xf32>, memref<64x128xbf16, 3>
      frisk.copy %1[], %arg1[%arg2 * 64, %arg3 * 128] {dstExtents = array<i64: 64, 128>, srcExtents = array<i64: 64, 128>} : memref<64x128xbf16, 3>, memref<256x256xbf16, 1>
      frisk.end
    }
    frisk.end
  }
}
