"""Pins for the oracle (oracle/), which is the checker of every GPU parity test.

What pins each part:
  * tile addressing: element offset = coord * tile shape (known answers of
    test/xt/to_nova.mlir:142-144)
  * sharing rule: the C executor's closed form against oracle/interp.py, a
    literal restatement of lib/xt/XTSerialize.cpp's reuse cache, on programs
    whose shared index moves along the shared axes (so the rule matters); a
    planted wrong rule is shown to fail the same check
  * conv halo slices: the three known answers of test/xt/to_nova.mlir:148-156,
    and the oracle's zero-padding conv equals "slice + pad + valid conv"
  * arithmetic: closed forms (numpy float64), brute force on tiny shapes,
    special cases (identity matrix, delta filter, one-hot softmax row)
  * conversions: f16 against numpy, bf16 against bit-exact expectations
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf, interp
from xtile_amd import kernels as K


def run_c(text, bufs, threads=2):
    bufs = [np.array(b, copy=True) for b in bufs]
    oracle.run(text, bufs, threads)
    return bufs


def run_py(text, bufs):
    bufs = [np.array(b, copy=True) for b in bufs]
    interp.run(text, bufs)
    return bufs


# -- tile addressing -------------------------------------------------------------


@pytest.mark.parametrize("coords,start", [((0, 2), (0, 32)), ((1, 2), (16, 32))])
def test_tile_offset_known_answers(coords, start):
    """to_nova.mlir:142-144: tile coordinate (0,2) of a 16x16 tile starts at
    element [0, 32]; (1,2) at [16, 32]."""
    text = f"""
func.func @t(%src: memref<64x48xf32>, %dst: memref<16x16xf32>) attributes {{xt.grid = array<i32: 1, 1, 1>}} {{
  %a = arith.constant {coords[0]} : i32
  %b = arith.constant {coords[1]} : i32
  %z = arith.constant 0 : i32
  %0 = xt.load(%src, %a, %b) : (memref<64x48xf32>, i32, i32) -> tensor<16x16xf32>
  xt.store(%0, %dst, %z, %z) : (tensor<16x16xf32>, memref<16x16xf32>, i32, i32) -> ()
  func.return
}}"""
    src = np.arange(64 * 48, dtype=np.float32).reshape(64, 48)
    out = run_c(text, [src, np.zeros((16, 16), np.float32)])[1]
    r, c = start
    np.testing.assert_array_equal(out, src[r : r + 16, c : c + 16])


# -- sharing rule ------------------------------------------------------------------

SHARED_PROG = """
func.func @s(%src: memref<64x64xf32>, %dst: memref<GRIDZx64x64xf32>) attributes {xt.grid = array<i32: GX, GY, GZ>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%src, %bid#0, %bid#1) {shared = K : i64} : (memref<64x64xf32>, i32, i32) -> tensor<16x16xf32>
  xt.store(%0, %dst, %bid#2, %bid#0, %bid#1) : (tensor<16x16xf32>, memref<GRIDZx64x64xf32>, i32, i32, i32) -> ()
  func.return
}"""


def _shared_program(k, grid):
    gx, gy, gz = grid
    # rank-3 destination so every block stores to its own tile
    return (
        SHARED_PROG.replace("GRIDZ", str(gz))
        .replace("GX", str(gx))
        .replace("GY", str(gy))
        .replace("GZ", str(gz))
        .replace("K :", f"{k} :")
        .replace("tensor<16x16xf32>, memref", "tensor<1x16x16xf32>, memref")
    )


def _shared_text(k, grid):
    gx, gy, gz = grid
    return f"""
func.func @s(%src: memref<64x64xf32>, %dst: memref<{gz}x64x64xf32>) attributes {{xt.grid = array<i32: {gx}, {gy}, {gz}>}} {{
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%src, %bid#0, %bid#1) {{shared = {k} : i64}} : (memref<64x64xf32>, i32, i32) -> tensor<16x16xf32>
  %1 = xt.reshape(%0) : tensor<16x16xf32> -> tensor<1x16x16xf32>
  xt.store(%1, %dst, %bid#2, %bid#0, %bid#1) : (tensor<1x16x16xf32>, memref<{gz}x64x64xf32>, i32, i32, i32) -> ()
  func.return
}}"""


@pytest.mark.parametrize("k", [0, 1, 2])
@pytest.mark.parametrize("grid", [(2, 2, 1), (3, 2, 2), (4, 4, 1), (1, 3, 2)])
def test_sharing_closed_form_equals_literal_serialize(k, grid):
    text = _shared_text(k, grid)
    rng = np.random.default_rng(0)
    src = rng.normal(size=(64, 64)).astype(np.float32)
    dst = np.full((grid[2], 64, 64), -7.0, np.float32)
    c_out = run_c(text, [src, dst])[1]
    py_out = run_py(text, [src, dst])[1]
    np.testing.assert_array_equal(c_out, py_out)
    # every block's stored tile is the group leader's tile
    for z in range(grid[2]):
        for y in range(grid[1]):
            for x in range(grid[0]):
                lx = 0 if k >= 1 else x
                ly = 0 if k >= 2 else y
                np.testing.assert_array_equal(
                    c_out[z, x * 16 : x * 16 + 16, y * 16 : y * 16 + 16],
                    src[lx * 16 : lx * 16 + 16, ly * 16 : ly * 16 + 16],
                )


def test_planted_wrong_sharing_rule_is_caught():
    """A plausible mistake - forcing axes <= k instead of < k - must fail the
    literal-serialize comparison above."""
    text = _shared_text(1, (2, 2, 1))
    rng = np.random.default_rng(0)
    src = rng.normal(size=(64, 64)).astype(np.float32)
    dst = np.zeros((1, 64, 64), np.float32)
    want = run_py(text, [src, dst])[1]
    wrong = np.zeros_like(want)
    for y in range(2):
        for x in range(2):
            wrong[0, x * 16 : x * 16 + 16, y * 16 : y * 16 + 16] = src[0:16, 0:16]  # forced x and y
    assert not np.array_equal(wrong, want)


# -- conv halo slices ----------------------------------------------------------------


@pytest.mark.parametrize(
    "idx,start,size,pads",
    [
        ((1, 1), (31, 63), (34, 66), (0, 0, 0, 0)),
        ((0, 0), (0, 0), (33, 65), (1, 1, 0, 0)),
        ((2, 2), (63, 127), (33, 65), (0, 0, 1, 1)),
    ],
)
def test_conv_slice_known_answers(idx, start, size, pads):
    """test/xt/to_nova.mlir:148-156 (source 96x192, tile 32x64, 3x3, pad 1)."""
    h = cf.conv_slice(96, idx[0], 32, 3, 1, 1, 1)
    w = cf.conv_slice(192, idx[1], 64, 3, 1, 1, 1)
    assert (h[0], w[0]) == start
    assert (h[1], w[1]) == size
    assert (h[2], w[2], h[3], w[3]) == pads  # [top, left, bottom, right]


def test_conv_out_dim_rule():
    assert cf.conv_out_dim(56, 3, 1, 1, 1, 1) == 56
    assert cf.conv_out_dim(34, 3, 0, 0, 1, 1) == 32
    assert cf.conv_out_dim(9, 3, 1, 1, 2, 2) == 4


@pytest.mark.parametrize("idx", [(0, 0), (1, 1), (2, 2), (1, 0)])
def test_oracle_conv_equals_slice_pad_valid_conv(idx):
    """The oracle's zero-outside formula equals the reference lowering: load the
    halo slice, zero-pad it by the slice pads, run a valid convolution."""
    H, W, C, CO, TH, TW = 24, 48, 8, 4, 8, 16
    rng = np.random.default_rng(1)
    x = rng.integers(-3, 4, (1, H, W, C)).astype(np.float16)
    f = rng.integers(-2, 3, (3, 3, C, CO)).astype(np.float16)
    text = str(K.conv2d(1, H, W, C, CO, 3, 3, TH, TW))
    out = run_c(text, [x, f, np.zeros((1, H, W, CO), np.float32)])[2]
    hs = cf.conv_slice(H, idx[0], TH, 3, 1, 1, 1)
    ws = cf.conv_slice(W, idx[1], TW, 3, 1, 1, 1)
    sl = x[0, hs[0] : hs[0] + hs[1], ws[0] : ws[0] + ws[1]].astype(np.float64)
    padded = np.pad(sl, ((hs[2], hs[3]), (ws[2], ws[3]), (0, 0)))
    valid = np.zeros((TH, TW, CO))
    for kh in range(3):
        for kw in range(3):
            valid += padded[kh : kh + TH, kw : kw + TW] @ f[kh, kw].astype(np.float64)
    got = out[0, idx[0] * TH : idx[0] * TH + TH, idx[1] * TW : idx[1] * TW + TW]
    np.testing.assert_array_equal(got, valid.astype(np.float32))


# -- arithmetic ----------------------------------------------------------------------


def test_add_is_ieee_f32():
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (64, 128)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 128)).astype(np.float32)
    c = run_c(str(K.add(64, 128, 32, 64)), [a, b, np.zeros_like(a)])[2]
    assert np.array_equal(c, a + b)
    assert np.array_equal(c, b + a)


def test_softmax_closed_form_and_invariants():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 2, (32, 512)).astype(np.float32)
    x[3] = -1e4
    x[3, 17] = 5.0  # one-hot row
    y = run_c(str(K.softmax(32, 512, 4)), [x, np.zeros_like(x)])[1]
    ref = cf.softmax_rows(x)
    assert np.max(np.abs(y - ref) / np.maximum(ref, 1e-30)) < 2e-6
    np.testing.assert_allclose(y.sum(axis=1), 1.0, atol=1e-6)
    assert y[3, 17] == 1.0 and np.count_nonzero(y[3]) == 1
    assert np.all((y >= 0) & (y <= 1))


def test_softmax_is_x_times_reciprocal_of_sum():
    """x / r is traced as mul(x, reciprocal(r)): the oracle must round like that."""
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (4, 64)).astype(np.float32)
    y = run_c(str(K.softmax(4, 64, 4)), [x, np.zeros_like(x)])[1]
    d = x - x.max(axis=1, keepdims=True)  # f32 subtraction, as traced
    e = np.exp(d.astype(np.float64)).astype(np.float32)  # correctly rounded expf
    s = np.zeros((4, 1), np.float32)
    for j in range(64):
        s += e[:, j : j + 1]
    want = e * (np.float32(1.0) / s)
    np.testing.assert_allclose(y, want, rtol=4e-7, atol=0)  # ~3 ulp: expf vs rounded exp


def test_matmul_closed_form_identity_and_brute_force():
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (128, 128)).astype(np.float16)
    eye = np.eye(128, dtype=np.float16)
    text = str(K.matmul_f16(128, 128, 128, 64, 64))
    out = run_c(text, [a, eye, np.zeros((128, 128), np.float32)])[2]
    np.testing.assert_array_equal(out, a.astype(np.float32))
    b = rng.uniform(-1, 1, (128, 128)).astype(np.float16)
    out = run_c(text, [a, b, np.zeros((128, 128), np.float32)])[2]
    ref = cf.matmul(a, b)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-7
    # brute force on a corner
    for i, j in [(0, 0), (5, 77), (127, 127)]:
        bf = sum(float(a[i, k]) * float(b[k, j]) for k in range(128))
        assert abs(out[i, j] - bf) <= 1e-6 * max(1.0, abs(bf))


def test_planted_transposed_operand_is_caught():
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (64, 64)).astype(np.float16)
    b = rng.uniform(-1, 1, (64, 64)).astype(np.float16)
    out = run_c(str(K.matmul_f16(64, 64, 64, 64, 64)), [a, b, np.zeros((64, 64), np.float32)])[2]
    wrong = cf.matmul(a, b.T)
    assert np.linalg.norm(out - wrong) / np.linalg.norm(wrong) > 1e-1


def test_conv_delta_filter_and_closed_form():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 0.1, (2, 8, 16, 32)).astype(np.float16)
    delta = np.zeros((3, 3, 32, 32), np.float16)
    delta[1, 1] = np.eye(32, dtype=np.float16)  # center tap identity
    text = str(K.conv2d(2, 8, 16, 32, 32, 3, 3, 4, 8))
    out = run_c(text, [x, delta, np.zeros((2, 8, 16, 32), np.float32)])[2]
    np.testing.assert_array_equal(out, x.astype(np.float32))
    f = rng.normal(0, 0.1, (3, 3, 32, 32)).astype(np.float16)
    out = run_c(text, [x, f, np.zeros((2, 8, 16, 32), np.float32)])[2]
    ref = cf.conv2d_nhwc(x, f, 1, 1)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-7
    # shifted-tap delta: out[h, w] = x[h-1, w+1] (zero outside)
    sh = np.zeros_like(delta)
    sh[0, 2] = np.eye(32, dtype=np.float16)
    out = run_c(text, [x, sh, np.zeros((2, 8, 16, 32), np.float32)])[2]
    want = np.zeros_like(out)
    want[:, 1:, :-1] = x[:, :-1, 1:].astype(np.float32)
    np.testing.assert_array_equal(out, want)


def test_conv_brute_force_tiny_and_strided():
    rng = np.random.default_rng(6)
    text = """
func.func @c(%x: memref<1x7x9x2xf16>, %f: memref<3x3x2x3xf16>, %y: memref<1x3x4x3xf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %w = xt.load(%f, %z, %z, %z, %z) : (memref<3x3x2x3xf16>, i32, i32, i32, i32) -> tensor<3x3x2x3xf16>
  %o = xt.load_conv2d(%x, %w, %z, %z, %z, %z) {dilation = array<i64: 2, 1>, group = 1 : i64, pad = array<i64: 1, 2, 1, 2>, stride = array<i64: 2, 2>} : (memref<1x7x9x2xf16>, tensor<3x3x2x3xf16>, i32, i32, i32, i32) -> tensor<1x3x4x3xf32>
  xt.store(%o, %y, %z, %z, %z, %z) : (tensor<1x3x4x3xf32>, memref<1x3x4x3xf32>, i32, i32, i32, i32) -> ()
  func.return
}"""
    x = rng.integers(-4, 5, (1, 7, 9, 2)).astype(np.float16)
    f = rng.integers(-3, 4, (3, 3, 2, 3)).astype(np.float16)
    out = run_c(text, [x, f, np.zeros((1, 3, 4, 3), np.float32)])[2]
    want = np.zeros((1, 3, 4, 3))
    for oh in range(3):
        for ow in range(4):
            for o in range(3):
                acc = 0.0
                for kh in range(3):
                    for kw in range(3):
                        ih, iw = oh * 2 - 1 + kh * 2, ow * 2 - 2 + kw
                        if 0 <= ih < 7 and 0 <= iw < 9:
                            acc += sum(float(x[0, ih, iw, c]) * float(f[kh, kw, c, o]) for c in range(2))
                want[0, oh, ow, o] = acc
    np.testing.assert_array_equal(out, want.astype(np.float32))
    np.testing.assert_array_equal(
        out, cf.conv2d_nhwc(x, f, 1, 2, (2, 2), (2, 1), out_hw=(3, 4)).astype(np.float32)
    )
    np.testing.assert_array_equal(run_py(text, [x, f, np.zeros((1, 3, 4, 3), np.float32)])[2], out)


def test_planted_dropped_pad_is_caught():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (1, 8, 8, 32)).astype(np.float16)
    f = rng.normal(0, 1, (3, 3, 32, 16)).astype(np.float16)
    out = run_c(str(K.conv2d(1, 8, 8, 32, 16, 3, 3, 4, 8)), [x, f, np.zeros((1, 8, 8, 16), np.float32)])[2]
    wrong = cf.conv2d_nhwc(x, f, 0, 0, out_hw=(8, 8))
    assert np.linalg.norm(out - wrong) / np.linalg.norm(out) > 1e-1


# -- element conversions ----------------------------------------------------------------


def test_f16_conversions_match_numpy():
    lib = oracle.lib()
    rng = np.random.default_rng(8)
    vals = np.concatenate(
        [
            rng.normal(0, 100, 4000).astype(np.float32),
            rng.normal(0, 1e-5, 2000).astype(np.float32),
            np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6e-8, 3e-8, 2.9802322e-08, np.inf], np.float32),
        ]
    )
    with np.errstate(over="ignore"):
        expected = vals.astype(np.float16).view(np.uint16)
    for v, bits in zip(vals, expected):
        assert lib.xo_f32_to_f16(float(v)) == bits, v
    for bits in range(0, 65536, 7):
        h = np.uint16(bits).view(np.float16)
        if np.isnan(h):
            continue
        assert lib.xo_f16_to_f32(bits) == np.float32(h)


def test_bf16_conversions():
    lib = oracle.lib()
    # known answers: exact, round down, tie to even (down), tie to even (up)
    cases = {
        1.0: 0x3F80,
        np.float32(np.uint32(0x3F808000).view(np.float32)): 0x3F80,  # 1 + 2^-8: tie, even stays
        np.float32(np.uint32(0x3F818000).view(np.float32)): 0x3F82,  # tie, odd rounds up
        np.float32(np.uint32(0x3F80FFFF).view(np.float32)): 0x3F81,
        -2.0: 0xC000,
    }
    for v, bits in cases.items():
        assert lib.xo_f32_to_bf16(float(v)) == bits
        assert oracle.f32_to_bf16_bits(np.array([v], np.float32))[0] == bits
    rng = np.random.default_rng(9)
    x = rng.normal(0, 0.02, 5000).astype(np.float32)
    numpy_bits = oracle.f32_to_bf16_bits(x)
    assert all(lib.xo_f32_to_bf16(float(v)) == b for v, b in zip(x[:500], numpy_bits[:500]))
    back = oracle.bf16_bits_to_f32(numpy_bits)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2.0**-8)


def test_oracle_i8_matmul_epilogue_matches_numpy():
    """kernels/matmul.py: exact integer products, nearest-f32 conversion, f32
    multiply then f32 add (no fused multiply-add), ftoi half-to-even with
    saturation; a planted round-half-away rule is caught."""
    rng = np.random.default_rng(6)
    m, n, k = 64, 192, 256
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    s = (rng.uniform(0.5, 2.0, (1, n)) / (np.sqrt(k) * 64)).astype(np.float32)
    bias = rng.uniform(-20, 20, (1, n)).astype(np.float32)
    out = run_c(str(K.matmul_i8(m, n, k)), [a, b, np.zeros((m, n), np.int8), s, bias])[2]
    f = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    y = ((f * s).astype(np.float32) + bias).astype(np.float32)
    np.testing.assert_array_equal(out, np.clip(np.rint(y), -128, 127).astype(np.int8))
    half_away = np.clip(np.sign(y) * np.floor(np.abs(y) + 0.5), -128, 127).astype(np.int8)
    ties = np.abs(y - np.trunc(y)) == 0.5
    if ties.any():
        assert not np.array_equal(out, half_away)
    # ftoi special cases through a single-element program
    vals = np.array([[0.5, 1.5, 2.5, -0.5, -1.5, 127.4, 127.6, -128.6, 1e9, -1e9, np.nan, -0.0]], np.float32)
    text = """
func.func @f(%x: memref<1x12xf32>, %y: memref<1x12xi8>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%x, %z, %z) : (memref<1x12xf32>, i32, i32) -> tensor<1x12xf32>
  %1 = xt.ftoi(%0) : tensor<1x12xf32> -> tensor<1x12xi8>
  xt.store(%1, %y, %z, %z) : (tensor<1x12xi8>, memref<1x12xi8>, i32, i32) -> ()
  func.return
}"""
    got = run_c(text, [vals, np.zeros((1, 12), np.int8)])[1]
    np.testing.assert_array_equal(got[0], np.array([0, 2, 2, 0, -2, 127, 127, -128, 127, -128, 0, 0], np.int8))


# -- general tile programs (the GPU tile interpreter's op set) ---------------------


def test_oracle_layernorm_matches_float64_closed_form():
    """Row layernorm (reduce, broadcast subtract, square, reduce, rsqrt, gamma,
    beta): the oracle's broadcasts and reductions against numpy float64."""
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1.5, (128, 64)).astype(np.float32)
    g = rng.normal(1, 0.2, (1, 64)).astype(np.float32)
    b = rng.normal(0, 0.2, (1, 64)).astype(np.float32)
    inv_n = np.full((1, 1), 1.0 / 64, np.float32)
    eps = np.full((1, 1), 1e-5, np.float32)
    y = run_c(str(K.layernorm(128, 64, 64)), [x, g, b, inv_n, eps, np.zeros_like(x)])[5]
    xd = x.astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    var = ((xd - mu) ** 2).mean(axis=1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * g + b
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-5)
    # a planted error in the checker (gamma and beta swapped) is caught
    bad = (xd - mu) / np.sqrt(var + 1e-5) * b + g
    assert np.max(np.abs(y - bad)) > 0.1


def test_oracle_column_softmax_and_bias_add():
    rng = np.random.default_rng(12)
    x = rng.normal(0, 2, (64, 128)).astype(np.float32)
    y = run_c(str(K.column_softmax(64, 128, 32)), [x, np.zeros_like(x)])[1]
    ref = cf.softmax_rows(x.T).T
    assert np.max(np.abs(y - ref) / np.maximum(ref, 1e-30)) < 2e-6
    np.testing.assert_allclose(y.sum(axis=0), 1.0, atol=1e-6)
    v = rng.normal(0, 1, (1, 256)).astype(np.float32)
    a = rng.normal(0, 1, (128, 256)).astype(np.float32)
    out = run_c(str(K.bias_add(128, 256)), [a, v, np.zeros_like(a)])[2]
    assert np.array_equal(out, a + v)  # IEEE f32 add, broadcast along rows


def test_oracle_unary_chain_transpose_and_reshape():
    """cos -> sin -> rsqrt -> sigmoid -> tanh -> silu, reshape, transpose of a
    rank-3 tile (the last two dims swap), against numpy."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl
    import xtile_amd as xt

    kernel, args, grid, db = programs(dsl)["unary_and_shape"]
    m = xt.convert(kernel, args=args, grid=grid, double_buffering=db)
    rng = np.random.default_rng(13)
    x = rng.uniform(-1, 1, (8, 8)).astype(np.float32)
    t = rng.normal(0, 1, (2, 3, 4)).astype(np.float32)
    bufs = run_c(str(m), [x, np.zeros((8, 8), np.float32), np.zeros((4, 16), np.float32), t,
                          np.zeros((2, 4, 3), np.float32)])
    v = x.astype(np.float64)
    v = np.sin(np.cos(v))
    v = 1 / np.sqrt(v)
    v = 1 / (1 + np.exp(-v))
    v = np.tanh(v)
    v = v / (1 + np.exp(-v))
    np.testing.assert_allclose(bufs[1], v, rtol=2e-6, atol=0)
    assert np.array_equal(bufs[2], bufs[1].reshape(4, 16))
    assert np.array_equal(bufs[4], t.transpose(0, 2, 1))


def test_oracle_mma_is_acc_plus_product():
    """test/python/dsl_convert.py:229-247 (xt.mma, i8 operands, f32
    accumulator): the exact float64 sum rounded once to f32; a planted
    accumulator-dropping checker is caught."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl
    import xtile_amd as xt

    kernel, args, grid, db = programs(dsl)["compute_ops"]
    m = xt.convert(kernel, args=args, grid=grid, double_buffering=db)
    rng = np.random.default_rng(14)
    a = rng.integers(-128, 128, (16, 32), dtype=np.int8)
    b = rng.integers(-128, 128, (32, 8), dtype=np.int8)
    acc = rng.normal(0, 1000, (16, 8)).astype(np.float32)
    out = run_c(str(m), [a, b, acc, np.zeros((16, 8), np.float32)])[3]
    exact = a.astype(np.float64) @ b.astype(np.float64) + acc.astype(np.float64)
    assert np.array_equal(out, exact.astype(np.float32))
    assert not np.array_equal(out, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))


def test_oracle_two_sided_broadcast_and_narrow_stores():
    """numpy broadcasting on both operands (lib/xt/XTOps.cpp:104-145); f16
    stores equal numpy's nearest-even astype, i8 stores saturate."""
    import xtile_amd as xt

    text = """
func.func @bc(%a: memref<8x1xf32>, %b: memref<1x16xf32>, %c: memref<8x16xf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%a, %z, %z) : (memref<8x1xf32>, i32, i32) -> tensor<8x1xf32>
  %1 = xt.load(%b, %z, %z) : (memref<1x16xf32>, i32, i32) -> tensor<1x16xf32>
  %2 = xt.sub(%0, %1) : tensor<8x1xf32>, tensor<1x16xf32> -> tensor<8x16xf32>
  xt.store(%2, %c, %z, %z) : (tensor<8x16xf32>, memref<8x16xf32>, i32, i32) -> ()
  func.return
}"""
    rng = np.random.default_rng(15)
    a = rng.normal(0, 1, (8, 1)).astype(np.float32)
    b = rng.normal(0, 1, (1, 16)).astype(np.float32)
    out = run_c(str(xt.parse(text)), [a, b, np.zeros((8, 16), np.float32)])[2]
    assert np.array_equal(out, a - b)
    assert not np.array_equal(out, b.T - a.T)  # operands swapped
    add = """
func.func @n(%a: memref<4x64xT>, %b: memref<4x64xT>, %c: memref<4x64xT>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%a, %z, %z) : (memref<4x64xT>, i32, i32) -> tensor<4x64xT>
  %1 = xt.load(%b, %z, %z) : (memref<4x64xT>, i32, i32) -> tensor<4x64xT>
  %2 = xt.add(%0, %1) : tensor<4x64xT>, tensor<4x64xT> -> tensor<4x64xT>
  xt.store(%2, %c, %z, %z) : (tensor<4x64xT>, memref<4x64xT>, i32, i32) -> ()
  func.return
}"""
    x = rng.normal(0, 3000, (4, 64)).astype(np.float16)
    y = rng.normal(0, 3000, (4, 64)).astype(np.float16)
    x[0, :3] = [65504, 1.0, 2048]
    y[0, :3] = [16, 2.0**-11, 1]
    out = run_c(str(xt.parse(add.replace("xT", "xf16"))), [x, y, np.zeros_like(x)])[2]
    with np.errstate(over="ignore"):  # 65504 + 16 rounds to inf, as it should
        want = (x.astype(np.float32) + y.astype(np.float32)).astype(np.float16)
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))
    i = rng.integers(-128, 128, (4, 64), dtype=np.int8)
    j = rng.integers(-128, 128, (4, 64), dtype=np.int8)
    out = run_c(str(xt.parse(add.replace("xT", "xi8"))), [i, j, np.zeros_like(i)])[2]
    assert np.array_equal(out, np.clip(i.astype(np.int32) + j.astype(np.int32), -128, 127).astype(np.int8))
