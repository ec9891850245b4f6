"""GPU parity at the special values IEEE arithmetic fixes, at the C1 and C2
benchmark shapes.

add (xtile/dsl.py:324-325): f32 addition is exactly specified by IEEE 754,
so the GPU must agree bit for bit with the oracle and with numpy on signed
zeros, subnormals (no flush to zero), overflow to infinity, infinities and
NaN.  NaN payloads are not specified: NaN is compared by class.

row softmax (kernels/softmax.py:13-18: x - max, exp, sum, x * (1/sum)):
  * a one-hot row (one 0, the rest -1e4): exp(-1e4) is 0 in f32, so the
    result is exactly 1 at the hot element and exactly 0 elsewhere;
  * a constant row: every e^0 is 1, the sum is 4096 exactly and 1/4096 is
    2^-12, so every element is exactly 2^-12;
  * -inf entries: exp(-inf) = 0 exactly;
  * an N(0, 20) row, whose exps underflow below the normal range;
  * an all -inf row, a row with +inf and a row with NaN: -inf - -inf,
    inf - inf and NaN propagate to a NaN sum, so every element is NaN;
  * a row of +-3e38 (x - max overflows to -inf) and a row of subnormals.
Bar: NaN where the oracle has NaN; where the oracle value is at least
FLT_MIN, relative error <= 1e-5 (the north star's softmax bar); where it is
below FLT_MIN (subnormal or zero, where the GPU's exp may round or flush
differently from the host's), absolute error <= FLT_MIN; exact values where
the mathematics fixes them (above).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import oracle_threads
from tests.gpu_util import run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu

FLT_MIN = np.float32(np.finfo(np.float32).tiny)
SUB = np.float32(1e-40)  # subnormal
MIN_SUB = np.float32(np.finfo(np.float32).smallest_subnormal)
FMAX = np.float32(np.finfo(np.float32).max)


def _same_bits_or_both_nan(got: np.ndarray, want: np.ndarray) -> None:
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), "NaN positions differ"
    ok = ~nan_w
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_add_special_values_c1_shape(cuda):
    """C1: 1024 x 1024, 32 x 64 tiles, special pairs placed in several tiles."""
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    pairs = [
        (0.0, -0.0), (-0.0, -0.0), (-0.0, 0.0), (0.0, 0.0),           # signed zeros
        (SUB, SUB), (-SUB, SUB / 2), (MIN_SUB, MIN_SUB), (MIN_SUB, -MIN_SUB),  # subnormal sums
        (FLT_MIN, -SUB), (FLT_MIN, -FLT_MIN / 2), (1.0, SUB), (SUB, -1e-38),   # normal / subnormal mixes
        (FMAX, FMAX), (-FMAX, -FMAX), (FMAX, -FMAX),                 # overflow, exact cancellation
        (np.inf, 1.0), (-np.inf, -np.inf), (np.inf, -np.inf),         # infinities, inf - inf
        (np.nan, 1.0), (1.0, np.nan), (np.nan, np.inf),               # NaN
    ]
    pa = np.array([p[0] for p in pairs], np.float32)
    pb = np.array([p[1] for p in pairs], np.float32)
    n = len(pairs)
    for r, c in [(0, 0), (31, 40), (32, 64), (517, 333), (1023, 1024 - n), (700, 960)]:
        a[r, c : c + n] = pa
        b[r, c : c + n] = pb
    # a whole tile of subnormal sums
    a[64:96, 128:192] = rng.uniform(-1, 1, (32, 64)).astype(np.float32) * SUB
    b[64:96, 128:192] = rng.uniform(-1, 1, (32, 64)).astype(np.float32) * SUB
    m = K.add(1024, 1024, 32, 64)
    host = [a, b, np.zeros_like(a)]
    got = run_gpu(m, host, ["f32"] * 3, cuda, case="add special values 1024x1024 tile 32x64")[2]
    want = run_oracle(m, host, oracle_threads())[2]
    with np.errstate(over="ignore", invalid="ignore"):
        ieee = a + b
    _same_bits_or_both_nan(want, ieee)  # the oracle is IEEE addition
    _same_bits_or_both_nan(got, want)
    # the properties the pairs were chosen for (placement at row 0, column 0)
    g = got[0, :n]
    bits = g.view(np.uint32)
    assert bits[0] == 0x00000000 and bits[1] == 0x80000000  # +0 + -0 = +0, -0 + -0 = -0
    assert bits[2] == 0 and bits[3] == 0
    assert g[4] == np.float32(2 * SUB) and 0 < g[4] < FLT_MIN  # subnormal sum, not flushed
    assert bits[6] == 2 and bits[7] == 0                        # 2 x smallest subnormal; x - x = +0
    assert np.isposinf(g[12]) and np.isneginf(g[13]) and bits[14] == 0
    assert np.isposinf(g[15]) and np.isneginf(g[16]) and np.isnan(g[17])
    assert np.all(np.isnan(g[18:21]))
    tile = got[64:96, 128:192]
    assert np.count_nonzero((tile != 0) & (np.abs(tile) < FLT_MIN)) > 1000  # subnormal results kept


def _softmax_special_rows(rng, cols):
    rows = []
    one_hot = np.full(cols, -1e4, np.float32)
    one_hot[17] = 0.0
    rows.append(("one_hot", one_hot))
    rows.append(("constant", np.full(cols, 3.0, np.float32)))
    r = rng.normal(0.0, 2.0, cols).astype(np.float32)
    r[::7] = -np.inf
    rows.append(("neg_inf_entries", r))
    rows.append(("wide_underflow", rng.normal(0.0, 20.0, cols).astype(np.float32)))
    rows.append(("all_neg_inf", np.full(cols, -np.inf, np.float32)))
    r = rng.normal(0.0, 2.0, cols).astype(np.float32)
    r[100] = np.inf
    rows.append(("pos_inf", r))
    r = rng.normal(0.0, 2.0, cols).astype(np.float32)
    r[2000] = np.nan
    rows.append(("nan", r))
    r = np.where(rng.uniform(size=cols) < 0.5, -3e38, 3e38).astype(np.float32)
    rows.append(("huge", r))
    rows.append(("subnormal", (rng.uniform(-1, 1, cols) * SUB).astype(np.float32)))
    return rows


def test_softmax_special_rows_c2_shape(cuda):
    """C2: 8192 x 4096, one 1 x 4096 row per Block, special rows at the start,
    the middle and the end of the array among N(0, 2) rows."""
    rows, cols = 8192, 4096
    rng = np.random.default_rng(2)
    x = rng.normal(0.0, 2.0, (rows, cols)).astype(np.float32)
    special = _softmax_special_rows(rng, cols)
    where = {}
    for base in (0, 4090, rows - len(special)):
        for i, (name, row) in enumerate(special):
            x[base + i] = row
            where.setdefault(name, []).append(base + i)
    m = K.softmax(rows, cols, 1)
    host = [x, np.zeros_like(x)]
    got = run_gpu(m, host, ["f32"] * 2, cuda, case="softmax special rows 8192x4096")[1]
    with np.errstate(invalid="ignore"):
        want = run_oracle(m, host, oracle_threads())[1]
    # NaN by class
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    normal = ok & (np.abs(want) >= FLT_MIN)
    tiny = ok & (np.abs(want) < FLT_MIN)
    rel = np.abs(got[normal] - want[normal]) / np.abs(want[normal])
    assert rel.max() <= 1e-5
    assert np.abs(got[tiny] - want[tiny]).max() <= FLT_MIN
    # what the mathematics fixes
    for r in where["one_hot"]:
        expect = np.zeros(cols, np.float32)
        expect[17] = 1.0
        assert np.array_equal(got[r], expect)
    for r in where["constant"] + where["subnormal"]:
        assert np.all(got[r] == np.float32(2.0**-12))
    for r in where["neg_inf_entries"]:
        assert np.all(got[r, ::7] == 0.0)
        assert abs(float(got[r].sum(dtype=np.float64)) - 1.0) <= 1e-5
    for r in where["all_neg_inf"] + where["pos_inf"] + where["nan"]:
        assert np.all(np.isnan(got[r]))
    for r in where["huge"]:
        big = x[r] > 0
        np.testing.assert_allclose(got[r][big], 1.0 / big.sum(), rtol=1e-6)
        assert np.all(got[r][~big] == 0.0)
    for r in where["wide_underflow"]:
        assert np.count_nonzero(want[r] < FLT_MIN) > 100  # the row does reach below the normal range
        assert abs(float(got[r].sum(dtype=np.float64)) - 1.0) <= 1e-5
    # every ordinary row still sums to one
    plain = np.ones(rows, bool)
    for rs in where.values():
        plain[rs] = False
    np.testing.assert_allclose(got[plain].sum(axis=1), 1.0, rtol=0, atol=1e-5)


def _ftoi_reference(y: np.ndarray) -> np.ndarray:
    """astype(int8) as xt.ftoi defines it: NaN -> 0, round half to even,
    saturate to [-128, 127]."""
    with np.errstate(invalid="ignore"):
        r = np.rint(np.nan_to_num(y.astype(np.float64), nan=0.0, posinf=1e300, neginf=-1e300))
    return np.clip(r, -128, 127).astype(np.int8)


@pytest.mark.parametrize("mn", [512, 384])
def test_matmul_i8_epilogue_special_values(cuda, mn):
    """kernels/matmul.py's epilogue t * scale + bias -> astype(int8) at the
    values that decide a float -> i8 conversion: scale or bias NaN, +-inf, -0,
    huge (past the i32 range), and exact halves (A, B in {-1, 0, 1} and scale
    0.5 make most outputs k + 0.5, which must round to even).  512 x 512 runs
    on the 256 x 256 DMA kernel, 384 x 384 on the 128 x 128 staged kernel.
    Checked bit for bit against the oracle and against the closed form above
    (the products are exact small integers, so t * s + b is one f32 multiply
    and one f32 add)."""
    m_ = n_ = mn
    k_ = 256
    rng = np.random.default_rng(11)
    a = rng.integers(-1, 2, (m_, k_), dtype=np.int8)
    b = rng.integers(-1, 2, (k_, n_), dtype=np.int8)
    s = np.full((1, n_), 0.5, np.float32)
    bias = np.zeros((1, n_), np.float32)
    special = [
        (np.nan, 0.0), (np.inf, 0.0), (-np.inf, 0.0), (0.0, np.inf), (0.0, -np.inf), (1.0, np.nan),
        (1.0, 3e38), (1.0, -3e38), (1e30, 0.0), (-1e30, 0.0), (-0.0, -0.0), (0.5, 0.5), (0.5, -0.5),
        (-0.5, 0.0), (0.25, 0.0), (1.5, 0.25), (3.0, 0.5), (1e-45, 0.0), (0.5, 127.5), (0.5, -128.5),
    ]
    for c0 in range(0, n_, 32):  # every 32 columns: every wave, tile and lane group
        for i, (sv, bv) in enumerate(special):
            s[0, c0 + i] = sv
            bias[0, c0 + i] = bv
    mod = K.matmul_i8(m_, n_, k_, 64, 64)
    c = np.zeros((m_, n_), np.int8)
    got = run_gpu(mod, [a, b, c, s, bias], ["i8", "i8", "i8", "f32", "f32"], cuda,
                  case=f"mm i8 epilogue special values {m_}x{n_}x{k_}")[2]
    want = run_oracle(mod, [a, b, c, s, bias], oracle_threads())[2]
    assert np.array_equal(want, got)
    acc = a.astype(np.int64) @ b.astype(np.int64)
    with np.errstate(invalid="ignore", over="ignore"):
        t = acc.astype(np.float32) * s
        y = (t + bias).astype(np.float32)
    assert np.array_equal(_ftoi_reference(y), got)
    # the ties really occur, and NaN columns give 0
    with np.errstate(invalid="ignore"):
        ties = (np.abs(y - np.floor(y)) == 0.5) & (np.abs(y) < 128)
    assert np.count_nonzero(ties) > m_ * n_ // 4
    assert np.all(got[:, 0] == 0) and np.all(got[:, 5] == 0)
