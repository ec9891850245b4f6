"""GPU parity of the tile interpreter (kernels/tilevm.hip) and of the staged
kernel that compiles the same lowering (csrc/staged.cpp) against the oracle.

Programs: the reference DSL test programs that are neither one of the four
benchmark families nor conv (unary ops, reshape, transpose, column reduce,
divide, the i8 mma program), the xt form of the reference's layernorm program,
a column softmax, a broadcast bias add, a rank-3 permute, f32 matmul, an
attention Block, small-tile i8 matmul epilogues, f16 / bf16 / i8 loads and
stores, and two-sided broadcasts.

Bars: IEEE f32 add / sub / mul / divide, pure data movement, narrow-type
conversions and exact i8 sums are bit-exact;
transcendental ops (GPU device libm against glibc) within 4e-6 relative;
reductions (a different summation order) within 1e-5 relative to the row
scale; f32 matmul within a Frobenius 1e-6.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.conftest import oracle_threads
from oracle import bf16_bits_to_f32, f32_to_bf16_bits
from tests.gpu_util import frob_rel, run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["staged", "interpreter"])
def vm_path(request, monkeypatch):
    """Every program here runs twice: compiled (the staged kernel, for the
    programs the fused layout declines) and on the interpreter itself
    (XTILE_AMD_STAGE=0)."""
    if request.param == "interpreter":
        monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    return request.param


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


# -- matmul / mma, casts, narrow types, two-sided broadcast ---------------------


def test_mma_i8_is_bit_exact(cuda):
    """test/python/dsl_convert.py:229-247: acc + A @ B with i8 A, B and an f32
    accumulator.  The i8 sum is exact and is rounded once with the accumulator,
    as in the oracle."""
    m = _golden("compute_ops")
    rng = np.random.default_rng(27)
    a = rng.integers(-128, 128, (16, 32), dtype=np.int8)
    b = rng.integers(-128, 128, (32, 8), dtype=np.int8)
    acc = rng.normal(0, 1000, (16, 8)).astype(np.float32)
    bufs = [a, b, acc, np.zeros((16, 8), np.float32)]
    got = run_gpu(m, bufs, ["i8", "i8", "f32", "f32"], cuda, case="mma i8")[3]
    want = run_oracle(m, bufs, 1)[3]
    assert np.array_equal(got, want)
    np.testing.assert_allclose(want, acc + a.astype(np.float64) @ b.astype(np.float64), rtol=1e-7)


@xt.kernel
def _f32_matmul(a, b, c, tm, tk, tn):
    i = xt.bid(0)
    j = xt.bid(1)
    x = xt.load(a, index=(i, 0), shape=(tm, tk))
    y = xt.load(b, index=(0, j), shape=(tk, tn), shared=1)
    xt.store(c, index=(i, j), tile=xt.matmul(x, y))


def test_f32_matmul(cuda):
    """The DSL's float32 matmul (xtile/dsl.py:369-374: matching dtypes keep
    theirs).  f32 sums in a different order: Frobenius 1e-6."""
    rng = np.random.default_rng(28)
    M, K, N, tm, tn = 96, 48, 80, 32, 40
    m = xt.convert(_f32_matmul, args=(xt.Array((M, K), xt.float32), xt.Array((K, N), xt.float32),
                                      xt.Array((M, N), xt.float32), tm, K, tn), grid=(M // tm, N // tn, 1),
                   double_buffering=False)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = rng.normal(0, 1, (K, N)).astype(np.float32)
    got = run_gpu(m, [a, b, np.zeros((M, N), np.float32)], ["f32"] * 3, cuda, case="f32 matmul")[2]
    want = run_oracle(m, [a, b, np.zeros((M, N), np.float32)], 1)[2]
    assert frob_rel(got, want) <= 1e-6


@xt.kernel
def _attention(q, k, v, o, tq, d, nk):
    i = xt.bid(0)
    qt = xt.load(q, index=(i, 0), shape=(tq, d))
    kt = xt.load(k, index=(0, 0), shape=(nk, d), shared=1)
    vt = xt.load(v, index=(0, 0), shape=(nk, d), shared=1)
    # the DSL transposes rank-3 tiles (xtile/dsl.py transpose): K^T via reshapes
    ktt = xt.reshape(xt.transpose(xt.reshape(kt, shape=(1, nk, d))), shape=(d, nk))
    s = xt.matmul(qt, ktt)
    p = xt.exp(s - xt.max(s, axis=1))
    p = p / xt.sum(p, axis=1)
    xt.store(o, index=(i, 0), tile=xt.matmul(p, vt))


def test_attention_block(cuda):
    """softmax(Q K^T) V for a 16-row query tile in one Block: matmul,
    transpose, row max / sum and broadcast ops chained in LDS."""
    rng = np.random.default_rng(29)
    nq, nk, d, tq = 64, 32, 32, 16
    m = xt.convert(_attention, args=(xt.Array((nq, d), xt.float32), xt.Array((nk, d), xt.float32),
                                     xt.Array((nk, d), xt.float32), xt.Array((nq, d), xt.float32), tq, d, nk),
                   grid=(nq // tq, 1, 1), double_buffering=False)
    q = rng.normal(0, 0.5, (nq, d)).astype(np.float32)
    k = rng.normal(0, 0.5, (nk, d)).astype(np.float32)
    v = rng.normal(0, 1, (nk, d)).astype(np.float32)
    bufs = [q, k, v, np.zeros((nq, d), np.float32)]
    got = run_gpu(m, bufs, ["f32"] * 4, cuda, case="attention block")[3]
    want = run_oracle(m, bufs, 1)[3]
    assert frob_rel(got, want) <= 1e-5
    s = q.astype(np.float64) @ k.T.astype(np.float64)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    np.testing.assert_allclose(want, (p / p.sum(axis=1, keepdims=True)) @ v, rtol=0, atol=1e-5)


def test_small_tile_i8_matmul_epilogue_is_bit_exact(cuda, vm_path):
    """kernels/matmul.py's program with 16 x 8 tiles (below the MFMA GEMM's
    64 x 64): i8 x i8, * scale + bias, astype(int8)."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    kern = programs(dsl)["matmul_int8_epilogue"][0]
    M, N, Kd, tm, tn = 32, 24, 40, 16, 8
    m = xt.convert(kern, args=(xt.Array((M, Kd), xt.int8), xt.Array((Kd, N), xt.int8), xt.Array((M, N), xt.int8),
                               xt.Array((1, N), xt.float32), xt.Array((1, N), xt.float32), tm, tn, Kd),
                   grid=(M // tm, N // tn, 1), double_buffering=True)
    assert xt.plan(m)["kernel"].startswith("staged" if vm_path == "staged" else "tile_vm")
    rng = np.random.default_rng(30)
    a = rng.integers(-128, 128, (M, Kd), dtype=np.int8)
    b = rng.integers(-128, 128, (Kd, N), dtype=np.int8)
    s = (rng.uniform(0.5, 2.0, (1, N)) / (np.sqrt(Kd) * 64)).astype(np.float32)
    bias = rng.uniform(-20, 20, (1, N)).astype(np.float32)
    bufs = [a, b, np.zeros((M, N), np.int8), s, bias]
    got = run_gpu(m, bufs, ["i8", "i8", "i8", "f32", "f32"], cuda, case="small-tile i8 epilogue")[2]
    want = run_oracle(m, bufs, 1)[2]
    assert np.array_equal(got, want)
    assert np.any(want == 127) and np.any(want == -128) and len(np.unique(want)) > 50


_NARROW = """
func.func @narrow(%a: memref<8x64xT>, %b: memref<8x64xT>, %c: memref<8x64xT>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%a, %z, %z) : (memref<8x64xT>, i32, i32) -> tensor<8x64xT>
  %1 = xt.load(%b, %z, %z) : (memref<8x64xT>, i32, i32) -> tensor<8x64xT>
  %2 = xt.add(%0, %1) : tensor<8x64xT>, tensor<8x64xT> -> tensor<8x64xT>
  xt.store(%2, %c, %z, %z) : (tensor<8x64xT>, memref<8x64xT>, i32, i32) -> ()
  func.return
}"""


def _f16_edges(rng):
    """Sums that round to even at ties, overflow to inf, land in the subnormal
    range, and NaN."""
    a = rng.normal(0, 4, (8, 64)).astype(np.float16)
    b = rng.normal(0, 4, (8, 64)).astype(np.float16)
    # 65520 ties past the largest half -> inf; 1 + 2^-11 ties -> 1; subnormal sums; inf - inf; NaN
    a[0, :8] = [65504, 65504, 1.0, 2.0**-24, 2.0**-14, -2.0**-24, np.inf, np.nan]
    b[0, :8] = [16, 65504, 2.0**-11, 2.0**-24, -2.0**-24, 0, -np.inf, 1]
    # above a tie rounds up; 2049 and 2051 tie to the even neighbours 2048 and 2052
    a[1, :4] = [1.0, 1.0, 2048, 2050]
    b[1, :4] = [2.0**-11, 1.5 * 2.0**-11, 1, 1]
    return a, b


def _as_f32(x, et):
    return bf16_bits_to_f32(x) if et == "bf16" else x.astype(np.float32)


@pytest.mark.parametrize("fuse", ["1", "0"])
@pytest.mark.parametrize("et", ["f16", "bf16", "i8"])
def test_narrow_loads_and_stores_round_like_the_oracle(cuda, et, fuse, monkeypatch):
    """On the fused kernel and (XTILE_AMD_FUSE=0) on the interpreter."""
    monkeypatch.setenv("XTILE_AMD_FUSE", fuse)
    rng = np.random.default_rng(31)
    m = xt.parse(_NARROW.replace("xT", "x" + et))
    assert xt.plan(m)["kernel"].startswith("fused" if fuse == "1" else "tile_vm")
    if et == "f16":
        a, b = _f16_edges(rng)
    elif et == "bf16":
        a = f32_to_bf16_bits(rng.normal(0, 100, (8, 64)).astype(np.float32))
        b = f32_to_bf16_bits(rng.normal(0, 100, (8, 64)).astype(np.float32))
        a[0, :4] = f32_to_bf16_bits(np.array([3.0e38, 1.0, np.nan, -0.0], np.float32))
        b[0, :4] = f32_to_bf16_bits(np.array([3.0e38, 2.0**-8, 1.0, -0.0], np.float32))
    else:
        a = rng.integers(-128, 128, (8, 64), dtype=np.int8)
        b = rng.integers(-128, 128, (8, 64), dtype=np.int8)
    c = np.zeros_like(a)
    got = run_gpu(m, [a, b, c], [et] * 3, cuda, case=f"narrow add {et}")[2]
    want = run_oracle(m, [a, b, c], 1)[2]
    if et == "i8":  # saturating sums
        assert np.array_equal(got, want)
        assert np.array_equal(want, np.clip(a.astype(np.int32) + b.astype(np.int32), -128, 127).astype(np.int8))
        return
    # bit-exact, except that a NaN's sign and payload are not compared
    nan_g, nan_w = np.isnan(_as_f32(got, et)), np.isnan(_as_f32(want, et))
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got.view(np.uint16)[~nan_w], want.view(np.uint16)[~nan_w])
    if et == "f16":
        w = want.astype(np.float32)
        assert np.isinf(w[0, 0]) and np.isinf(w[0, 1]) and w[0, 2] == 1.0 and w[0, 3] == 2.0**-23
        assert w[0, 4] == 2.0**-14 - 2.0**-24 and np.isnan(w[0, 6]) and np.isnan(w[0, 7])
        assert list(w[1, :4]) == [1.0, 1.0 + 2.0**-10, 2048, 2052]


@pytest.mark.parametrize("fuse", ["1", "0"])
def test_two_sided_broadcast(cuda, fuse, monkeypatch):
    """(8, 1) - (1, 16) -> (8, 16) and a rank-1 operand (lib/xt/XTOps.cpp:104-145),
    on the fused kernel and on the interpreter."""
    monkeypatch.setenv("XTILE_AMD_FUSE", fuse)
    text = """
func.func @bc(%a: memref<8x1xf32>, %b: memref<1x16xf32>, %v: memref<16xf32>, %c: memref<8x16xf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%a, %z, %z) : (memref<8x1xf32>, i32, i32) -> tensor<8x1xf32>
  %1 = xt.load(%b, %z, %z) : (memref<1x16xf32>, i32, i32) -> tensor<1x16xf32>
  %2 = xt.load(%v, %z) : (memref<16xf32>, i32) -> tensor<16xf32>
  %3 = xt.sub(%0, %1) : tensor<8x1xf32>, tensor<1x16xf32> -> tensor<8x16xf32>
  %4 = xt.mul(%2, %3) : tensor<16xf32>, tensor<8x16xf32> -> tensor<8x16xf32>
  xt.store(%4, %c, %z, %z) : (tensor<8x16xf32>, memref<8x16xf32>, i32, i32) -> ()
  func.return
}"""
    m = xt.parse(text)
    assert xt.plan(m)["kernel"].startswith("fused" if fuse == "1" else "tile_vm")
    rng = np.random.default_rng(32)
    a = rng.normal(0, 1, (8, 1)).astype(np.float32)
    b = rng.normal(0, 1, (1, 16)).astype(np.float32)
    v = rng.normal(0, 1, (16,)).astype(np.float32)
    bufs = [a, b, v, np.zeros((8, 16), np.float32)]
    got = run_gpu(m, bufs, ["f32"] * 4, cuda, case="two-sided broadcast")[3]
    want = run_oracle(m, bufs, 1)[3]
    assert np.array_equal(got, want)
    assert np.array_equal(want, v * (a - b))
