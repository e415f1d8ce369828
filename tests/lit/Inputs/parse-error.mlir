module attributes {frisk.target = "gfx950"} {
  frisk.kernel @k(memref<64xf32, 1>) {
  ^bb0(%arg0: memref<64xf32, 1>):
    frisk.fill %undefined {value = 1.000000e+00 : f32} : memref<64xf32, 1>
    frisk.end
  }
}
