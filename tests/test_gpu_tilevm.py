"""GPU parity of the tile interpreter (kernels/tilevm.hip) against the oracle.

Programs: the reference DSL test programs that are neither one of the four
benchmark families nor matmul / conv (unary ops, reshape, transpose, column
reduce, divide), the xt form of the reference's layernorm program, a column
softmax, a broadcast bias add and a rank-3 permute.

Bars: IEEE f32 add / sub / mul / divide and pure data movement are bit-exact;
transcendental ops (GPU device libm against glibc) within 4e-6 relative;
reductions (a different summation order) within 1e-5 relative to the row
scale.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.conftest import oracle_threads
from tests.gpu_util import run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu


def _golden(name):
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    k, args, grid, db = programs(dsl)[name]
    return xt.convert(k, args=args, grid=grid, double_buffering=db)


def test_unary_chain_reshape_transpose(cuda):
    m = _golden("unary_and_shape")
    rng = np.random.default_rng(21)
    x = rng.uniform(-1, 1, (8, 8)).astype(np.float32)
    t = rng.normal(0, 1, (2, 3, 4)).astype(np.float32)
    bufs = [x, np.zeros((8, 8), np.float32), np.zeros((4, 16), np.float32), t, np.zeros((2, 4, 3), np.float32)]
    got = run_gpu(m, bufs, ["f32"] * 5, cuda, case="unary_and_shape")
    want = run_oracle(m, bufs, oracle_threads())
    np.testing.assert_allclose(got[1], want[1], rtol=4e-6, atol=0)
    assert np.array_equal(got[2], got[1].reshape(4, 16))
    assert np.array_equal(got[4], want[4])
    assert np.array_equal(got[4], t.transpose(0, 2, 1))


def test_column_reduce_and_divide(cuda):
    rng = np.random.default_rng(22)
    m = _golden("column_reduce")
    x = rng.normal(0, 1, (8, 8)).astype(np.float32)
    got = run_gpu(m, [x, np.zeros((1, 8), np.float32)], ["f32"] * 2, cuda, case="column_reduce")[1]
    want = run_oracle(m, [x, np.zeros((1, 8), np.float32)], 1)[1]
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * np.abs(x).sum(axis=0).max())
    m = _golden("divide_kernel")
    a = rng.normal(0, 1, (8, 8)).astype(np.float32)
    d = rng.uniform(0.5, 2, (8, 1)).astype(np.float32)
    got = run_gpu(m, [a, d, np.zeros_like(a)], ["f32"] * 3, cuda, case="divide")[2]
    want = run_oracle(m, [a, d, np.zeros_like(a)], 1)[2]
    assert np.array_equal(got, want)  # x * (1 / d), both correctly rounded


@pytest.mark.parametrize("rows,cols,trow", [(128, 64, 64), (1024, 256, 32), (96, 48, 16)])
def test_layernorm(cuda, rows, cols, trow):
    rng = np.random.default_rng(23)
    m = K.layernorm(rows, cols, trow)
    x = rng.normal(0, 1.5, (rows, cols)).astype(np.float32)
    g = rng.normal(1, 0.2, (1, cols)).astype(np.float32)
    b = rng.normal(0, 0.2, (1, cols)).astype(np.float32)
    inv_n = np.full((1, 1), 1.0 / cols, np.float32)
    eps = np.full((1, 1), 1e-5, np.float32)
    bufs = [x, g, b, inv_n, eps, np.zeros_like(x)]
    got = run_gpu(m, bufs, ["f32"] * 6, cuda, case=f"layernorm {rows}x{cols}/{trow}")[5]
    want = run_oracle(m, bufs, oracle_threads())[5]
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("rows,cols,tcol", [(64, 128, 32), (100, 96, 32)])
def test_column_softmax(cuda, rows, cols, tcol):
    rng = np.random.default_rng(24)
    m = K.column_softmax(rows, cols, tcol)
    x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
    got = run_gpu(m, [x, np.zeros_like(x)], ["f32"] * 2, cuda, case=f"column softmax {rows}x{cols}")[1]
    want = run_oracle(m, [x, np.zeros_like(x)], oracle_threads())[1]
    assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
    np.testing.assert_allclose(got.sum(axis=0), 1.0, atol=1e-5)


def test_bias_add_is_bit_exact(cuda):
    rng = np.random.default_rng(25)
    m = K.bias_add(128, 256)
    a = rng.normal(0, 1, (128, 256)).astype(np.float32)
    v = rng.normal(0, 1, (1, 256)).astype(np.float32)
    got = run_gpu(m, [a, v, np.zeros_like(a)], ["f32"] * 3, cuda, case="bias add")[2]
    assert np.array_equal(got, a + v)


def test_permute_rank3(cuda):
    text = """
func.func @p(%a: memref<4x6x10xf32>, %b: memref<10x4x6xf32>) attributes {xt.grid = array<i32: 2, 2, 2>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%a, %bid#0, %bid#1, %bid#2) : (memref<4x6x10xf32>, i32, i32, i32) -> tensor<2x3x5xf32>
  %1 = xt.permute(%0) {permutation = [2, 0, 1]} : tensor<2x3x5xf32> -> tensor<5x2x3xf32>
  xt.store(%1, %b, %bid#2, %bid#0, %bid#1) : (tensor<5x2x3xf32>, memref<10x4x6xf32>, i32, i32, i32) -> ()
  func.return
}"""
    m = xt.parse(text)
    rng = np.random.default_rng(26)
    a = rng.normal(0, 1, (4, 6, 10)).astype(np.float32)
    got = run_gpu(m, [a, np.zeros((10, 4, 6), np.float32)], ["f32"] * 2, cuda, case="permute")[1]
    want = run_oracle(m, [a, np.zeros((10, 4, 6), np.float32)], 1)[1]
    assert np.array_equal(got, want)
    assert np.array_equal(got, a.transpose(2, 0, 1))
