"""GPU parity of the staged kernel (csrc/staged.cpp): tile programs that the
register-resident fused kernel declines - matmul / mma on MFMA, transposes and
permutes, values of several shapes - compiled per program, against the oracle
and against the tile interpreter (XTILE_AMD_STAGE=0) on the same inputs.

Bars: exact i8 sums (mma, the i8 matmul epilogue) bit-exact; f16 / bf16
operands (exact products, f32 sums) and f32 operands (f32 MFMA) within a
Frobenius 1e-5 of the oracle's double sums; softmax rows within 1e-5 of the
float64 closed form.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from oracle import f32_to_bf16_bits
from tests.conftest import oracle_threads
from tests.gpu_util import frob_rel, run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu


def _attention_inputs(rng, heads, nq, nk, d, qk):
    q = rng.normal(0, 0.5, (heads, nq, d)).astype(np.float32)
    k = rng.normal(0, 0.5, (heads, nk, d)).astype(np.float32)
    v = rng.normal(0, 1.0, (heads, nk, d)).astype(np.float32)
    if qk == "f16":
        q, k = q.astype(np.float16), k.astype(np.float16)
    elif qk == "bf16":
        q, k = f32_to_bf16_bits(q), f32_to_bf16_bits(k)
    return q, k, v


def _closed_form(q, k, v, qk):
    from oracle import bf16_bits_to_f32

    if qk == "bf16":
        q, k = bf16_bits_to_f32(q), bf16_bits_to_f32(k)
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    s = q @ np.swapaxes(k, 1, 2)
    p = np.exp(s - s.max(axis=2, keepdims=True))
    return (p / p.sum(axis=2, keepdims=True)) @ v


@pytest.mark.parametrize(
    "heads,nq,nk,d,tq,qk",
    [(2, 128, 64, 64, 64, "f16"),     # whole 32 x 32 MFMA tiles
     (3, 96, 40, 24, 32, "f16"),      # ragged: N = 40, K = 24 (the f16 K step of 16 padded)
     (2, 64, 128, 64, 64, "bf16"),
     (2, 48, 33, 20, 16, "f32"),      # M = 16 rows of a 32-row tile, odd key count
     (1, 64, 64, 128, 64, "f16")],    # d = 128
)
def test_attention_block(cuda, monkeypatch, heads, nq, nk, d, tq, qk):
    """softmax(Q K^T) V (xtile_amd.kernels.attention): the staged kernel, the
    tile interpreter and the oracle agree; the oracle agrees with float64."""
    dt = {"f16": xt.float16, "bf16": xt.bfloat16, "f32": xt.float32}[qk]
    rng = np.random.default_rng(31)
    q, k, v = _attention_inputs(rng, heads, nq, nk, d, qk)
    bufs = [q, k, v, np.zeros((heads, nq, d), np.float32)]
    dts = [qk, qk, "f32", "f32"]
    m = K.attention(heads, nq, nk, d, tq, qk=dt)
    plan = xt.plan(m)["kernel"]
    assert plan.startswith("staged") and "mfma=" in plan
    got = run_gpu(m, bufs, dts, cuda, case=f"attention {heads}x{nq}x{nk}x{d} tq={tq} {qk}")[3]
    want = run_oracle(m, bufs, oracle_threads())[3]
    assert frob_rel(got, want) <= 1e-5
    np.testing.assert_allclose(want, _closed_form(q, k, v, qk), rtol=0, atol=2e-5)
    monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    mi = K.attention(heads, nq, nk, d, tq, qk=dt)
    assert xt.plan(mi)["kernel"].startswith("tile_vm")
    interp = run_gpu(mi, bufs, dts, cuda, case="attention on the interpreter")[3]
    assert frob_rel(got, interp) <= 1e-5


def test_reference_mma_program_is_bit_exact(cuda):
    """The reference's mma program (test/python/dsl_convert.py:236-247:
    [16, 32] x [32, 8] int8 + a float32 accumulator) on the i8 MFMA: exact
    i32 sums, the accumulator added once, as the oracle rounds."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    kern, args, grid, db = programs(dsl)["compute_ops"]
    m = xt.convert(kern, args=args, grid=grid, double_buffering=db)
    assert "mfma=i8" in xt.plan(m)["kernel"]
    rng = np.random.default_rng(32)
    a = rng.integers(-128, 128, (16, 32), dtype=np.int8)
    b = rng.integers(-128, 128, (32, 8), dtype=np.int8)
    acc = rng.normal(0, 100, (16, 8)).astype(np.float32)
    bufs = [a, b, acc, np.zeros((16, 8), np.float32)]
    got = run_gpu(m, bufs, ["i8", "i8", "f32", "f32"], cuda, case="reference mma")[3]
    want = run_oracle(m, bufs, 1)[3]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@xt.kernel
def _matmul_then_ops(a, b, bias, out, tm, tn, tk):
    i = xt.bid(0)
    j = xt.bid(1)
    x = xt.load(a, index=(i, 0), shape=(tm, tk))
    w = xt.load(b, index=(0, j), shape=(tk, tn), shared=1)
    c = xt.load(bias, index=(0, j), shape=(1, tn), shared=1)
    t = xt.add(xt.matmul(x, w), c)
    t = xt.silu(t)
    r = xt.sum(t, axis=0)
    xt.store(out, index=(i, j), tile=xt.mul(t, r))


@pytest.mark.parametrize(
    "dt,m_,n_,k_,tm,tn",
    [("f16", 256, 192, 96, 64, 64), ("bf16", 128, 256, 64, 32, 128), ("f32", 96, 80, 40, 48, 40),
     ("f16", 40, 24, 24, 20, 12)],   # 20 x 12 tiles, K = 24: every guard
)
def test_matmul_followed_by_ops(cuda, dt, m_, n_, k_, tm, tn):
    """matmul + bias row, silu, a column sum broadcast back: the matmul's
    result feeds ops of several shapes in one Block."""
    xdt = {"f16": xt.float16, "bf16": xt.bfloat16, "f32": xt.float32}[dt]
    m = xt.convert(_matmul_then_ops, args=(xt.Array((m_, k_), xdt), xt.Array((k_, n_), xdt),
                                          xt.Array((1, n_), xt.float32), xt.Array((m_, n_), xt.float32), tm, tn, k_),
                   grid=(m_ // tm, n_ // tn, 1), double_buffering=False)
    assert xt.plan(m)["kernel"].startswith("staged")
    rng = np.random.default_rng(33)
    a = rng.normal(0, 0.3, (m_, k_)).astype(np.float32)
    b = rng.normal(0, 0.3, (k_, n_)).astype(np.float32)
    if dt == "f16":
        a, b = a.astype(np.float16), b.astype(np.float16)
    elif dt == "bf16":
        a, b = f32_to_bf16_bits(a), f32_to_bf16_bits(b)
    bias = rng.normal(0, 0.5, (1, n_)).astype(np.float32)
    bufs = [a, b, bias, np.zeros((m_, n_), np.float32)]
    got = run_gpu(m, bufs, [dt, dt, "f32", "f32"], cuda, case=f"matmul then ops {dt} {m_}x{n_}x{k_}")[3]
    want = run_oracle(m, bufs, oracle_threads())[3]
    assert frob_rel(got, want) <= 1e-5


@xt.kernel
def _matmul_then_row_norm(a, b, gamma, beta, inv_n, eps, out, rstd, tm, tn, tk):
    i = xt.bid(0)
    j = xt.bid(1)
    x = xt.load(a, index=(i, 0), shape=(tm, tk))
    w = xt.load(b, index=(0, j), shape=(tk, tn), shared=1)
    g = xt.load(gamma, index=(0, j), shape=(1, tn), shared=1)
    be = xt.load(beta, index=(0, j), shape=(1, tn), shared=1)
    n = xt.load(inv_n, index=(0, 0), shape=(1, 1), shared=1)
    e = xt.load(eps, index=(0, 0), shape=(1, 1), shared=1)
    t = xt.matmul(x, w)
    xc = xt.sub(t, xt.mul(xt.sum(t, axis=1), n))
    r = xt.rsqrt(xt.add(xt.mul(xt.sum(xt.mul(xc, xc), axis=1), n), e))
    xt.store(rstd, index=(i, j), tile=r)
    xt.store(out, index=(i, j), tile=xt.add(xt.mul(xt.mul(xc, r), g), be))


@pytest.mark.parametrize(
    "dt,m_,n_,k_,tm,tn",
    [("f16", 256, 128, 64, 64, 64),     # 4 lanes a row, one pass
     ("f32", 64, 48, 40, 32, 24),       # 8 lanes a row of 24: 3 elements a lane, scalar LDS accesses
     ("bf16", 256, 128, 32, 128, 64),   # 2 lanes a row of 64
     ("f32", 512, 16, 32, 512, 8),      # 512 rows of 8: a lane a row, two passes
     ("f16", 64, 256, 32, 16, 256)],    # 16 lanes a row of 256
)
def test_matmul_then_row_normalisation(cuda, monkeypatch, dt, m_, n_, k_, tm, tn):
    """matmul, then a layernorm along the result's rows with gamma / beta
    column vectors and (1, 1) scalars, storing the rows' 1/std as well: the
    row reductions and the ops around them run as one register step (a row
    segment); the staged kernel, the interpreter and the oracle agree."""
    xdt = {"f16": xt.float16, "bf16": xt.bfloat16, "f32": xt.float32}[dt]
    nt = n_ // tn

    def build():
        return xt.convert(_matmul_then_row_norm,
                          args=(xt.Array((m_, k_), xdt), xt.Array((k_, n_), xdt), xt.Array((1, n_), xt.float32),
                                xt.Array((1, n_), xt.float32), xt.Array((1, 1), xt.float32),
                                xt.Array((1, 1), xt.float32), xt.Array((m_, n_), xt.float32),
                                xt.Array((m_, nt), xt.float32), tm, tn, k_),
                          grid=(m_ // tm, nt, 1), double_buffering=False)

    m = build()
    assert xt.plan(m)["kernel"].startswith("staged")
    rng = np.random.default_rng(37)
    a = rng.normal(0, 0.3, (m_, k_)).astype(np.float32)
    b = rng.normal(0, 0.3, (k_, n_)).astype(np.float32)
    if dt == "f16":
        a, b = a.astype(np.float16), b.astype(np.float16)
    elif dt == "bf16":
        a, b = f32_to_bf16_bits(a), f32_to_bf16_bits(b)
    gamma = rng.normal(1, 0.2, (1, n_)).astype(np.float32)
    beta = rng.normal(0, 0.2, (1, n_)).astype(np.float32)
    bufs = [a, b, gamma, beta, np.full((1, 1), 1.0 / tn, np.float32), np.full((1, 1), 1e-5, np.float32),
            np.zeros((m_, n_), np.float32), np.zeros((m_, nt), np.float32)]
    dts = [dt, dt, "f32", "f32", "f32", "f32", "f32", "f32"]
    got = run_gpu(m, bufs, dts, cuda, case=f"matmul then row norm {dt} {m_}x{n_}x{k_} tiles {tm}x{tn}")
    want = run_oracle(m, bufs, oracle_threads())
    assert frob_rel(got[6], want[6]) <= 1e-5
    assert frob_rel(got[7], want[7]) <= 1e-5
    monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    mi = build()
    assert xt.plan(mi)["kernel"].startswith("tile_vm")
    interp = run_gpu(mi, bufs, dts, cuda, case="row norm on the interpreter")
    assert frob_rel(got[6], interp[6]) <= 1e-5
    assert frob_rel(got[7], interp[7]) <= 1e-5


def test_staged_and_interpreter_agree_on_the_i8_epilogue(cuda, monkeypatch):
    """kernels/matmul.py's program with 16 x 8 tiles (below the GEMM
    kernel's 64 x 64) and K = 72 (two i8 MFMA steps of 32, the second part
    padded): i8 x i8 exact, * scale + bias, astype(int8): the staged kernel,
    the interpreter and the oracle give the same bytes."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    kern = programs(dsl)["matmul_int8_epilogue"][0]
    M, N, Kd, tm, tn = 48, 40, 72, 16, 8

    def build():
        return xt.convert(kern, args=(xt.Array((M, Kd), xt.int8), xt.Array((Kd, N), xt.int8),
                                      xt.Array((M, N), xt.int8), xt.Array((1, N), xt.float32),
                                      xt.Array((1, N), xt.float32), tm, tn, Kd),
                          grid=(M // tm, N // tn, 1), double_buffering=True)

    m = build()
    assert "mfma=i8" in xt.plan(m)["kernel"]
    rng = np.random.default_rng(35)
    a = rng.integers(-128, 128, (M, Kd), dtype=np.int8)
    b = rng.integers(-128, 128, (Kd, N), dtype=np.int8)
    s = (rng.uniform(0.5, 2.0, (1, N)) / (np.sqrt(Kd) * 64)).astype(np.float32)
    bias = rng.uniform(-20, 20, (1, N)).astype(np.float32)
    bufs = [a, b, np.zeros((M, N), np.int8), s, bias]
    dts = ["i8", "i8", "i8", "f32", "f32"]
    got = run_gpu(m, bufs, dts, cuda, case="i8 epilogue staged")[2]
    want = run_oracle(m, bufs, 1)[2]
    assert np.array_equal(got, want)
    assert np.any(want == 127) and np.any(want == -128)
    monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    mi = build()
    assert xt.plan(mi)["kernel"].startswith("tile_vm")
    interp = run_gpu(mi, bufs, dts, cuda, case="i8 epilogue on the interpreter")[2]
    assert np.array_equal(got, interp)
