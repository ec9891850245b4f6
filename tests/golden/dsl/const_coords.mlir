func.func @const_coords(%input: memref<16x24xf32>, %output: memref<16x24xf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %zero = arith.constant 0 : i32
  %c1 = arith.constant 1 : i32
  %c2 = arith.constant 2 : i32
  %c3 = arith.constant 3 : i32

  %x = xt.load(%input, %c1, %c2) : (memref<16x24xf32>, i32, i32) -> tensor<4x8xf32>
  %x2 = xt.load(%input, %c3, %c1) : (memref<16x24xf32>, i32, i32) -> tensor<4x8xf32>
  %sum = xt.add(%x, %x2) : tensor<4x8xf32>, tensor<4x8xf32> -> tensor<4x8xf32>
  xt.store(%sum, %output, %c2, %zero) : (tensor<4x8xf32>, memref<16x24xf32>, i32, i32) -> ()
  func.return
}
