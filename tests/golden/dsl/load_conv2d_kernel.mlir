func.func @load_conv2d_kernel(%input: memref<1x34x66x128xi8>, %input2: memref<3x3x128x64xi8>, %output: memref<1x32x64x32xf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %zero = arith.constant 0 : i32

  %x = xt.load(%input2, %zero, %zero, %zero, %zero) : (memref<3x3x128x64xi8>, i32, i32, i32, i32) -> tensor<3x3x128x64xi8>
  %load_conv = xt.load_conv2d(%input, %x, %zero, %zero, %zero, %zero) {dilation = array<i64: 1, 1>, group = 1 : i64, pad = array<i64: 1, 1, 1, 1>, stride = array<i64: 1, 1>} : (memref<1x34x66x128xi8>, tensor<3x3x128x64xi8>, i32, i32, i32, i32) -> tensor<1x32x64x32xf32>
  xt.store(%load_conv, %output, %zero, %zero, %zero, %zero) : (tensor<1x32x64x32xf32>, memref<1x32x64x32xf32>, i32, i32, i32, i32) -> ()
  func.return
}
