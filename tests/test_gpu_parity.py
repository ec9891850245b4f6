"""GPU parity: every HIP kernel against the oracle on the same seeded inputs.

Bars: bit-exact for f32 add; max relative error <= 1e-5
for f32 softmax; Frobenius relative error <= 1e-3 for f16/bf16 matmul and conv.
Inputs follow the benchmark recipe: numpy PCG64, seed = config index.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from oracle import bf16_bits_to_f32, closed_form as cf, f32_to_bf16_bits
from tests.conftest import oracle_threads
from tests.gpu_util import frob_rel, run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu

SOFTMAX_RTOL = 1e-5
MM_FROB = 1e-3


# -- add (C1) ------------------------------------------------------------------


@pytest.mark.parametrize(
    "rows,cols,th,tw",
    [(1024, 1024, 32, 64), (64, 128, 32, 64), (96, 40, 32, 8), (33, 7, 11, 7), (1, 4, 1, 4),
     (128, 96, 64, 96), (256, 384, 64, 24), (64, 2048, 64, 2048)],
)
def test_add_bit_exact(cuda, rows, cols, th, tw):
    rng = np.random.default_rng(1)
    m = K.add(rows, cols, th, tw)
    a = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    b = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    c = np.zeros_like(a)
    got = run_gpu(m, [a, b, c], ["f32"] * 3, cuda, case=f"add {rows}x{cols} tile {th}x{tw}")[2]
    want = run_oracle(m, [a, b, c], oracle_threads())[2]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(want, a + b)


def test_add_rows_reference_program(cuda):
    """kernels/add.py form: 64-row full-width tiles, grid (rows/64, 1, 1)."""
    rng = np.random.default_rng(1)
    m = K.add_rows(256, 384, 64)
    a = rng.uniform(-1, 1, (256, 384)).astype(np.float32)
    b = rng.uniform(-1, 1, (256, 384)).astype(np.float32)
    got = run_gpu(m, [a, b, np.zeros_like(a)], ["f32"] * 3, cuda, case="add_rows")[2]
    assert np.array_equal(got, a + b)


@pytest.mark.parametrize("swap_b", [False, True])
@pytest.mark.parametrize("rows,cols,th,tw,grid", [(1024, 1024, 32, 64, (32, 16)), (96, 100, 24, 100, (4, 1)),
                                                   (128, 128, 32, 32, (4, 4)), (256, 64, 16, 16, (8, 4))])
def test_add_flat_and_tiled_forms(cuda, rows, cols, th, tw, grid, swap_b):
    """Programs whose tiles cover one contiguous run of every operand run as
    one flat stream (the planner says flat=N); a transposed Block index in B
    keeps the tiled kernel.  Both bit-exact against numpy on the covered
    region; elements outside it keep their prior contents."""
    from tests.test_plan import _ew_program

    if swap_b and (th != tw or rows != cols):
        pytest.skip("a transposed index needs square tiles over a square array")
    rng = np.random.default_rng(5)
    m = _ew_program(rows, cols, th, tw, grid, swap_b=swap_b)
    kernel = xt.plan(m)["kernel"]
    assert ("flat=" in kernel) == (not swap_b)
    a = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    b = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    c0 = rng.uniform(5, 6, (rows, cols)).astype(np.float32)
    got = run_gpu(m, [a, b, c0.copy()], ["f32"] * 3, cuda, case=f"add {rows}x{cols} tile {th}x{tw} swap={swap_b}")[2]
    want = c0.copy()
    for x in range(grid[0]):
        for y in range(grid[1]):
            bx, by = (y, x) if swap_b else (x, y)
            want[x * th:(x + 1) * th, y * tw:(y + 1) * tw] = (
                a[x * th:(x + 1) * th, y * tw:(y + 1) * tw] + b[bx * th:(bx + 1) * th, by * tw:(by + 1) * tw])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("op", ["sub", "mul"])
def test_sub_mul_bit_exact(cuda, op):
    text = f"""
func.func @k(%a: memref<64x96xf32>, %b: memref<64x96xf32>, %c: memref<64x96xf32>) attributes {{xt.grid = array<i32: 2, 3, 1>}} {{
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%a, %bid#0, %bid#1) : (memref<64x96xf32>, i32, i32) -> tensor<32x32xf32>
  %1 = xt.load(%b, %bid#0, %bid#1) : (memref<64x96xf32>, i32, i32) -> tensor<32x32xf32>
  %2 = xt.{op}(%0, %1) : tensor<32x32xf32>, tensor<32x32xf32> -> tensor<32x32xf32>
  xt.store(%2, %c, %bid#0, %bid#1) : (tensor<32x32xf32>, memref<64x96xf32>, i32, i32) -> ()
  func.return
}}"""
    m = xt.parse(text)
    rng = np.random.default_rng(7)
    a = rng.normal(size=(64, 96)).astype(np.float32)
    b = rng.normal(size=(64, 96)).astype(np.float32)
    got = run_gpu(m, [a, b, np.zeros_like(a)], ["f32"] * 3, cuda, case=op)[2]
    want = run_oracle(m, [a, b, np.zeros_like(a)], 2)[2]
    assert np.array_equal(got, want)


# -- softmax (C2) ----------------------------------------------------------------


@pytest.mark.parametrize(
    "rows,cols,trow",
    [(8192, 4096, 1), (128, 64, 64), (64, 4096, 2), (16, 1000, 4), (24, 8192, 1), (5, 3, 5),
     (9, 6144, 3), (16, 2048, 4), (6, 8192, 2)],
)
def test_softmax(cuda, rows, cols, trow):
    rng = np.random.default_rng(2)
    m = K.softmax(rows, cols, trow)
    x = rng.normal(0.0, 2.0, (rows, cols)).astype(np.float32)
    got = run_gpu(m, [x, np.zeros_like(x)], ["f32"] * 2, cuda, case=f"softmax {rows}x{cols}/{trow}")[1]
    want = run_oracle(m, [x, np.zeros_like(x)], oracle_threads())[1]
    rel = np.max(np.abs(got - want) / np.abs(want))
    assert rel <= SOFTMAX_RTOL
    np.testing.assert_allclose(got.sum(axis=1), 1.0, rtol=0, atol=1e-5)


# -- matmul (C3, C5) --------------------------------------------------------------


@pytest.mark.parametrize(
    "m_,n_,k_,tm,tn",
    [(4096, 4096, 4096, 128, 128), (256, 384, 192, 128, 128), (128, 192, 64, 64, 64), (512, 256, 512, 256, 128)],
)
def test_matmul_f16(cuda, m_, n_, k_, tm, tn):
    rng = np.random.default_rng(3)
    mod = K.matmul_f16(m_, n_, k_, tm, tn)
    a = rng.uniform(-1, 1, (m_, k_)).astype(np.float16)
    b = rng.uniform(-1, 1, (k_, n_)).astype(np.float16)
    c = np.zeros((m_, n_), np.float32)
    got = run_gpu(mod, [a, b, c], ["f16", "f16", "f32"], cuda, case=f"mm f16 {m_}x{n_}x{k_}")[2]
    want = run_oracle(mod, [a, b, c], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB
    assert frob_rel(want, cf.matmul(a, b)) <= 1e-6


@pytest.mark.parametrize(
    "m_,n_,k_,tm,tn", [(4096, 11008, 4096, 256, 128), (512, 640, 256, 256, 128), (256, 128, 128, 128, 64)]
)
def test_matmul_bf16(cuda, m_, n_, k_, tm, tn):
    rng = np.random.default_rng(5)
    mod = K.matmul_bf16(m_, n_, k_, tm, tn)
    a = f32_to_bf16_bits(rng.normal(0, 0.02, (m_, k_)).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.02, (k_, n_)).astype(np.float32))
    c = np.zeros((m_, n_), np.float32)
    got = run_gpu(mod, [a, b, c], ["bf16", "bf16", "f32"], cuda, case=f"mm bf16 {m_}x{n_}x{k_}")[2]
    ref = cf.matmul(bf16_bits_to_f32(a), bf16_bits_to_f32(b)) if m_ * n_ * k_ > 2**33 else None
    if ref is None:
        ref = run_oracle(mod, [a, b, c], oracle_threads())[2]
    assert frob_rel(got, ref) <= MM_FROB


@pytest.mark.parametrize(
    "dt,mn,k_,ftoi",
    [("f16", 256, 64, False), ("bf16", 256, 64, False), ("bf16", 512, 192, False), ("i8", 256, 128, False),
     ("i8", 512, 384, True), ("f16", 512, 64, True), ("bf16", 256, 128, True)],
)
def test_matmul_dma_kernel_short_k(cuda, dt, mn, k_, ftoi):
    """256 x 256 workgroup tiles (the DMA kernel; four waves for f16, eight
    for bf16 and i8) with K of two to six 64-byte stages, fewer than or just
    above the three stages its prologue puts in flight; f32 and i8 results."""
    rng = np.random.default_rng(12)
    dt_in = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}[dt]
    mod = _matmul_epilogue_program(mn, mn, k_, dt_in, True, True, ftoi)
    if dt == "i8":
        a, b, s, bi = _i8_inputs(rng, mn, mn, k_)
    else:
        a = rng.normal(0, 1, (mn, k_)).astype(np.float32)
        b = rng.normal(0, 1, (k_, mn)).astype(np.float32)
        a, b = (f32_to_bf16_bits(a), f32_to_bf16_bits(b)) if dt == "bf16" else (a.astype(np.float16), b.astype(np.float16))
        s = rng.uniform(0.05, 0.2, (1, mn)).astype(np.float32)
        bi = rng.uniform(-3, 3, (1, mn)).astype(np.float32)
    c = np.zeros((mn, mn), np.int8 if ftoi else np.float32)
    dts = [dt, dt, "i8" if ftoi else "f32", "f32", "f32"]
    got = run_gpu(mod, [a, b, c, s, bi], dts, cuda, case=f"mm dma {dt} {mn}x{mn}x{k_} ftoi={ftoi}")[2]
    want = run_oracle(mod, [a, b, c, s, bi], oracle_threads())[2]
    if dt == "i8":
        assert np.array_equal(got, want)
    elif ftoi:
        assert np.mean(got != want) < 1e-3 and np.max(np.abs(got.astype(int) - want.astype(int))) <= 1
    else:
        assert frob_rel(got, want) <= MM_FROB


# -- conv2d (C4) -------------------------------------------------------------------


@pytest.mark.parametrize(
    "n,h,w,cin,cout,th,tw",
    [(32, 56, 56, 64, 64, 4, 56), (2, 8, 16, 32, 16, 4, 8), (1, 7, 7, 64, 32, 7, 7), (3, 12, 20, 32, 128, 2, 10), (2, 6, 10, 96, 16, 3, 5)],
)
def test_conv2d_f16(cuda, n, h, w, cin, cout, th, tw):
    rng = np.random.default_rng(4)
    mod = K.conv2d(n, h, w, cin, cout, 3, 3, th, tw)
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float16)
    f = rng.normal(0, 0.1, (3, 3, cin, cout)).astype(np.float16)
    o = np.zeros((n, h, w, cout), np.float32)
    got = run_gpu(mod, [x, f, o], ["f16", "f16", "f32"], cuda, case=f"conv {n}x{h}x{w}x{cin}->{cout}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,dil,dt",
    [
        (2, 16, 16, 64, 64, 3, 3, 2, 8, (1, 1, 1, 1), (2, 2), (1, 1), "f16"),
        (2, 12, 12, 32, 48, 3, 3, 4, 12, (2, 2, 2, 2), (1, 1), (2, 2), "f16"),
        (1, 10, 14, 32, 32, 5, 5, 2, 14, (2, 2, 2, 2), (1, 1), (1, 1), "f16"),
        (2, 8, 16, 32, 80, 3, 3, 4, 16, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),
        (3, 9, 9, 96, 32, 1, 1, 3, 9, (0, 0, 0, 0), (1, 1), (1, 1), "f16"),
        (2, 11, 13, 32, 64, 3, 3, 3, 7, (0, 1, 2, 1), (2, 2), (1, 1), "f16"),
        (2, 14, 14, 64, 64, 3, 3, 7, 14, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),
        (1, 8, 8, 32, 128, 3, 3, 4, 8, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),
        (2, 12, 12, 32, 64, 3, 3, 4, 12, (2, 2, 2, 2), (1, 1), (2, 2), "f16"),
        (5, 61, 16, 32, 32, 3, 3, 61, 16, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),
    ],
)
def test_conv2d_general(cuda, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, dil, dt):
    """Strides, dilations, asymmetric padding, 1x1 / 5x5 filters, Cout with a
    partial 32-channel N tile (48, 80) and bf16 operands.  Cout a multiple of
    32 takes the band kernel (the 5 x 61-row case has 305 rows over the CUs:
    two-row bands with a one-row band at the end of each image); the others
    take the per-unit kernel."""
    rng = np.random.default_rng(5)
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xt.bfloat16 if dt == "bf16" else xt.float16,
                   pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
    if dt == "bf16":
        x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    else:
        x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda,
                  case=f"conv {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{stride} d{dil} {dt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "n,h,w,cin,pad,stride,dil,dt",
    [
        (32, 56, 56, 64, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),   # C4: 256 bands of 7 rows, 32 per XCD
        (2, 14, 14, 64, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),
        (2, 16, 16, 64, (1, 1, 1, 1), (2, 2), (1, 1), "f16"),    # stride 2
        (2, 11, 13, 32, (0, 1, 2, 1), (2, 2), (1, 1), "f16"),    # Cin 32 (two K steps a tap), asymmetric pad
        (2, 12, 12, 32, (2, 2, 2, 2), (1, 1), (2, 2), "bf16"),   # dilation 2
        (3, 30, 17, 64, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),   # odd width: M tiles cross rows unevenly
        (1, 100, 9, 32, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),    # one-row bands, a single M tile
        (4, 40, 120, 64, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),   # 122-pixel halo rows
        (1, 5, 300, 64, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),    # 10 M tiles in a one-row band
    ],
)
def test_conv2d_band_kernel_shapes(cuda, n, h, w, cin, pad, stride, dil, dt):
    """3 x 3 convolutions to 64 channels (f16 / bf16, Cin 32 or 64, Blocks
    covering the output) on the band kernel: bands dealt to the XCDs in
    contiguous runs, M tiles that cross output rows unevenly, one-row bands,
    wide halo rows, strides, dilation and asymmetric padding, against the
    oracle."""
    rng = np.random.default_rng(12)
    kh = kw = 3
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    th = next(t for t in (4, 3, 2, 1) if oh % t == 0)
    mod = K.conv2d(n, h, w, cin, 64, kh, kw, th, ow, dtype=xt.bfloat16 if dt == "bf16" else xt.float16,
                   pad=pad, stride=stride, dilation=dil)
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (kh, kw, cin, 64)).astype(np.float32)
    if dt == "bf16":
        x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    else:
        x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.zeros((n, oh, ow, 64), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda, case=f"conv band {n}x{h}x{w}x{cin}->64 s{stride} d{dil} {dt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,dil,dt",
    [
        (2, 12, 12, 128, 128, 3, 3, 4, 12, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),   # 295 KB filter: M 288, 3 tiles
        (4, 16, 16, 128, 256, 3, 3, 8, 16, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),   # 8 x 2 = 16 workgroups (XCD runs)
        (2, 9, 11, 256, 256, 3, 3, 5, 6, (1, 1, 1, 1), (2, 2), (1, 1), "bf16"),    # stride 2: M = 60, one partial tile
        (1, 7, 7, 512, 128, 3, 3, 7, 7, (2, 2, 2, 2), (1, 1), (2, 2), "f16"),      # dilation 2, 144 K stages
        (3, 10, 10, 64, 256, 1, 1, 5, 10, (0, 0, 0, 0), (1, 1), (1, 1), "f16"),    # 1 x 1, Cout 256
        (2, 16, 16, 96, 128, 5, 5, 5, 15, (2, 1, 1, 2), (1, 1), (1, 1), "bf16"),   # Cin 96: three stages a tap, asymmetric pad
        (2, 14, 14, 256, 128, 3, 3, 4, 12, (0, 0, 0, 0), (1, 1), (1, 1), "f16"),   # no padding: 12 x 12 outputs
        (2, 12, 12, 256, 64, 3, 3, 4, 12, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),    # Cout 64: 256 x 64 tiles
        (2, 10, 10, 160, 192, 3, 3, 5, 10, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),  # Cout 192: three 64-channel tiles
        (2, 12, 12, 256, 32, 3, 3, 4, 12, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),    # Cout 32: half a 64-channel tile
        (2, 14, 14, 48, 64, 3, 3, 7, 14, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),     # Cin 48: taps padded to 64 channels
        (2, 16, 16, 16, 40, 3, 3, 4, 8, (1, 1, 1, 1), (2, 2), (1, 1), "bf16"),     # Cin 16, Cout 40, stride 2
        (3, 9, 9, 1024, 48, 1, 1, 3, 9, (0, 0, 0, 0), (1, 1), (1, 1), "f16"),      # 1 x 1, Cout 48
        (1, 11, 13, 24, 200, 5, 5, 11, 13, (2, 2, 2, 2), (1, 1), (1, 1), "bf16"),  # Cin 24, Cout 200 (4 tiles, last 8 wide)
        (24, 14, 14, 512, 512, 3, 3, 2, 14, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),  # 148 tiles, 144 stages: K in halves
        (2, 10, 10, 192, 256, 3, 3, 5, 10, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),   # deep: 64 x 128 tiles, 3 128-byte stages a tap
        (8, 14, 14, 256, 256, 3, 3, 2, 14, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),  # C9's layer at batch 8: 50 deep tiles, K split
        (32, 14, 14, 256, 256, 3, 3, 2, 14, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),  # C9's layer: 196 deep tiles, rotated K walks
    ],
)
def test_conv2d_igemm(cuda, monkeypatch, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, dil, dt):
    """Filters too large for the band kernel's LDS (Cin * Cout * taps * 2
    bytes above ~150 KB) with Cout a multiple of 64 take the implicit-GEMM
    kernel (conv_igemm.hip; 128 x 128 tiles for Cout a multiple of 128, else
    256 x 64, and 64 x 128 tiles with 128-byte K stages for deep layers whose
    128 x 128 tiles would fill at most half the CUs, their DMA issued by
    eight loader waves and, for whole-K tiles, walked from a stage rotated
    per pixel tile): operands by DMA, the input gathered per tap, padding and
    rows past M read as zeros.  XTILE_AMD_CONV_IMAGE=0 keeps the shapes the
    resident-image kernel would take (C9's layer) on this one."""
    monkeypatch.setenv("XTILE_AMD_CONV_IMAGE", "0")
    rng = np.random.default_rng(9)
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xt.bfloat16 if dt == "bf16" else xt.float16,
                   pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
    if dt == "bf16":
        x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    else:
        x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda,
                  case=f"conv igemm {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{stride} d{dil} {dt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,th,tw,pad,stride,dil,dt,force",
    [
        (32, 14, 14, 256, 256, 3, 2, 14, (1, 1, 1, 1), (1, 1), (1, 1), "f16", ""),    # C9's layer: 256 workgroups, 7 M tiles
        (8, 12, 12, 256, 256, 3, 4, 12, (1, 1, 1, 1), (1, 1), (1, 1), "bf16", ""),    # 64 workgroups, 144 outputs: taken unforced
        (2, 14, 14, 256, 256, 3, 7, 14, (1, 1, 1, 1), (1, 1), (1, 1), "bf16", "1"),   # the same image, bf16, 16 workgroups
        (3, 16, 16, 64, 96, 3, 8, 16, (1, 1, 1, 1), (1, 1), (1, 1), "f16", "1"),      # 256 pixels (8 M tiles), one sub-chunk, Cout 96
        (2, 15, 15, 128, 64, 3, 8, 8, (1, 1, 1, 1), (2, 2), (1, 1), "f16", "1"),      # stride 2: 64 outputs of a 225-pixel image
        (2, 9, 9, 192, 32, 3, 5, 5, (0, 0, 0, 0), (1, 1), (2, 2), "bf16", "1"),       # dilation 2, no padding: 25 outputs, one tile
        (1, 10, 12, 64, 64, 5, 10, 12, (2, 1, 2, 1), (1, 1), (1, 1), "f16", "1"),     # 5 x 3 filter, asymmetric padding
        (2, 14, 14, 128, 64, 3, 12, 12, (0, 0, 0, 0), (1, 1), (1, 1), "f16", "1"),    # no padding: 144 of 196 pixels
        (2, 9, 9, 512, 64, 3, 9, 9, (1, 1, 1, 1), (1, 1), (1, 1), "bf16", "1"),       # 8 sub-chunks (133 KB of LDS)
    ],
)
def test_conv2d_resident_image(cuda, monkeypatch, n, h, w, cin, cout, kh, th, tw, pad, stride, dil, dt, force):
    """Deep layers whose image fits in LDS (Cin a multiple of 64, Cout of 32,
    a 3-wide filter, 128 to 256 outputs an image) take the resident-image
    kernel (conv_image.hip) when its workgroups, one per image and 32 output
    channels, fill at least a quarter of the CUs (C9's layer), and any such
    layer with XTILE_AMD_CONV_IMAGE=1: the image reaches LDS once in 64-channel
    sub-chunks, the filter streams through three stage buffers, four MFMA
    waves split K and add their partial sums through LDS; taps outside the
    image read a zero block."""
    if force:
        monkeypatch.setenv("XTILE_AMD_CONV_IMAGE", force)
    rng = np.random.default_rng(13)
    mod = K.conv2d(n, h, w, cin, cout, kh, 3, th, tw, dtype=xt.bfloat16 if dt == "bf16" else xt.float16,
                   pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * 2 - 1) // stride[1] + 1
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (kh, 3, cin, cout)).astype(np.float32)
    if dt == "bf16":
        x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    else:
        x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.full((n, oh, ow, cout), 7.0, np.float32)  # every output is written
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda,
                  case=f"conv image {n}x{h}x{w}x{cin}->{cout} k{kh}x3 s{stride} d{dil} {dt} force={force}")[2]
    want = run_oracle(mod, [x, f, np.zeros_like(o)], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


def test_conv2d_igemm_k_split_in_a_graph(cuda):
    """A K-split implicit-GEMM conv (52 tiles: K in 4 ranges, a zero-fill
    kernel, then partial sums added atomically) captured in a HIP graph and
    replayed three times, with eager work and synchronisations between the
    replays: every replay matches the eager launch and the oracle (the
    atomic addition order may change the last bits, so to a relative 1e-6)."""
    import torch

    rng = np.random.default_rng(12)
    n, h, w, cin, cout = 32, 7, 7, 512, 512
    mod = K.conv2d(n, h, w, cin, cout, 3, 3, 7, 7)
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float16)
    f = rng.normal(0, 0.1, (3, 3, cin, cout)).astype(np.float16)
    o = np.zeros((n, h, w, cout), np.float32)
    eager = run_gpu(mod, [x, f, o], ["f16", "f16", "f32"], cuda, case="conv igemm k-split eager")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(eager, want) <= MM_FROB
    print("[gpu] conv igemm k-split graph capture", flush=True)
    dx, df = torch.from_numpy(x).to(cuda), torch.from_numpy(f).to(cuda)
    do = torch.full((n, h, w, cout), 7.0, dtype=torch.float32, device=cuda)  # the zero fill must clear this
    stream = torch.cuda.Stream(device=cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        xt.launch(mod, dx, df, do, stream=stream)  # warm-up outside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            xt.launch(mod, dx, df, do, stream=stream)
    torch.cuda.synchronize()
    for r in range(3):
        do.fill_(float(r + 3))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = do.cpu().numpy()
        assert frob_rel(got, eager) <= 1e-6, r
        assert frob_rel(got, want) <= MM_FROB, r


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,first",
    [
        (2, 12, 12, 256, 128, 3, 3, 4, 12, (1, 1, 1, 1), (1, 1), "0"),  # 295 KB filter: 128 x 128 tiles
        (2, 8, 8, 320, 64, 3, 3, 8, 8, (1, 1, 1, 1), (1, 1), "0"),      # Cin 320: 256 x 64 tiles, 5 stages a tap
        (2, 13, 11, 128, 192, 3, 3, 7, 6, (1, 1, 1, 1), (2, 2), "0"),   # Cout 192: band declines (> 128)
        (1, 32, 64, 128, 64, 3, 3, 32, 64, (1, 1, 1, 1), (1, 1), "1"),  # kernels/conv2d.py, implicit GEMM first
        (2, 10, 10, 48, 80, 3, 3, 5, 10, (1, 1, 1, 1), (1, 1), "0"),    # Cin 48 padded to 64, Cout 80 (two tiles)
        (2, 12, 12, 272, 16, 3, 3, 4, 12, (1, 1, 1, 1), (1, 1), "0"),   # Cin 272 = 4 stages + 16, Cout 16
        (2, 9, 9, 384, 128, 3, 3, 9, 9, (1, 1, 1, 1), (1, 1), "0"),     # deep: 64 x 128 tiles, three 128-channel stages a tap
    ],
)
def test_conv2d_igemm_i8_bit_exact(cuda, monkeypatch, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, first):
    """i8 source and filter (the reference's own load_conv2d dtype) on the
    implicit-GEMM kernel: a K stage is 64 channels, filter fragments by
    ds_read_b64_tr_b8, exact i32 sums rounded to f32 once: bit-exact."""
    monkeypatch.setenv("XTILE_AMD_CONV_IGEMM", first)
    rng = np.random.default_rng(11)
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xt.int8, pad=pad, stride=stride)
    oh = (h + pad[0] + pad[2] - (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - (kw - 1) - 1) // stride[1] + 1
    x = rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8)
    f = rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8)
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], ["i8", "i8", "f32"], cuda,
                  case=f"conv igemm i8 {n}x{h}x{w}x{cin}->{cout} s{stride} first={first}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert np.array_equal(got, want)


@pytest.mark.parametrize(
    "n,h,w,cin,cout,th,tw,dt",
    [(32, 56, 56, 64, 64, 4, 56, "f16"), (3, 12, 20, 32, 128, 2, 10, "f16"), (2, 9, 7, 64, 64, 9, 7, "bf16")],
)
def test_conv2d_igemm_where_the_band_kernel_applies(cuda, monkeypatch, n, h, w, cin, cout, th, tw, dt):
    """XTILE_AMD_CONV_IGEMM=1 puts the implicit-GEMM kernel ahead of the band
    kernel: C4's shape (256 x 64 tiles, 392 workgroups) and small ones, 3 x 3
    "same" convolutions, against the oracle."""
    monkeypatch.setenv("XTILE_AMD_CONV_IGEMM", "1")
    rng = np.random.default_rng(10)
    mod = K.conv2d(n, h, w, cin, cout, 3, 3, th, tw, dtype=xt.bfloat16 if dt == "bf16" else xt.float16)
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (3, 3, cin, cout)).astype(np.float32)
    if dt == "bf16":
        x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    else:
        x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.zeros((n, h, w, cout), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda, case=f"conv igemm-first {n}x{h}x{w}x{cin}->{cout} {dt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,dil",
    [
        (1, 32, 64, 128, 64, 3, 3, 32, 64, (1, 1, 1, 1), (1, 1), (1, 1)),  # kernels/conv2d.py defaults
        (2, 16, 24, 64, 32, 3, 3, 8, 12, (1, 1, 1, 1), (2, 2), (1, 1)),
        (1, 20, 20, 64, 128, 3, 3, 4, 20, (2, 2, 2, 2), (1, 1), (2, 2)),
        (3, 9, 12, 64, 64, 1, 1, 3, 12, (0, 0, 0, 0), (1, 1), (1, 1)),
        (2, 11, 13, 64, 64, 3, 3, 3, 7, (0, 1, 2, 1), (2, 2), (1, 1)),
    ],
)
def test_conv2d_i8_bit_exact(cuda, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, dil):
    """The reference's own load_conv2d dtype (xtile/dsl.py:284-285): i8 source
    and filter, f32 result.  The i32 MFMA sum is exact and is rounded to f32
    once, as the oracle rounds its exact double sum, so the result is
    bit-exact."""
    rng = np.random.default_rng(6)
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xt.int8, pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    x = rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8)
    f = rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8)
    planted = kh == 3 and kw == 3 and cin == 128 and stride == (1, 1) and dil == (1, 1)
    if planted:
        # an odd sum above 2^24 at output (5, 5), channel 0: the i32 -> f32
        # conversion must round it (127 * 127 * 1151 + 126 * 127 = 18580481)
        x[0, 4:7, 4:7, :] = 127
        x[0, 4, 4, 0] = 126
        f[:, :, :, 0] = 127
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], ["i8", "i8", "f32"], cuda,
                  case=f"conv i8 {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{stride} d{dil}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    assert np.array_equal(got, want)
    if planted:
        assert want[0, 5, 5, 0] == np.float32(18580481.0) and float(want[0, 5, 5, 0]) != 18580481.0


def _conv_inputs(rng, dt, n, h, w, cin, cout, kh, kw):
    if dt == "i8":
        return (rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8),
                rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8))
    x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
    f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
    if dt == "bf16":
        return f32_to_bf16_bits(x), f32_to_bf16_bits(f)
    return x.astype(np.float16), f.astype(np.float16)


_DT = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,dil,dt",
    [
        (1, 8, 16, 3, 16, 3, 3, 4, 8, (1, 1, 1, 1), (1, 1), (1, 1), "i8"),     # RGB input: element gathers
        (1, 8, 8, 32, 32, 3, 3, 4, 8, (1, 1, 1, 1), (1, 1), (1, 1), "i8"),     # Cin < 64
        (1, 8, 8, 64, 256, 3, 3, 4, 8, (1, 1, 1, 1), (1, 1), (1, 1), "i8"),    # Cout > 128
        (2, 9, 11, 48, 40, 3, 3, 3, 11, (1, 1, 1, 1), (1, 1), (1, 1), "i8"),   # Cout % 32 != 0
        (1, 12, 12, 16, 64, 7, 7, 3, 3, (3, 3, 3, 3), (2, 2), (1, 1), "i8"),   # 7x7 stride 2, small tile
        (2, 10, 10, 8, 24, 3, 3, 5, 10, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),  # one K step spans two taps
        (1, 11, 13, 3, 5, 5, 5, 2, 7, (2, 2, 2, 2), (2, 2), (1, 1), "f16"),    # Cin 3, Cout 5
        (1, 10, 14, 64, 80, 5, 5, 2, 14, (2, 2, 2, 2), (1, 1), (1, 1), "f16"),  # filter beyond LDS
        (1, 9, 9, 20, 36, 3, 3, 4, 5, (2, 0, 1, 2), (1, 2), (2, 1), "bf16"),   # Cin % 8 != 0, odd everything
    ],
)
def test_conv2d_generic_kernel(cuda, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, dil, dt):
    """Shapes outside the band and persistent kernels (Cin not a multiple of
    32 or 64, Cout not a multiple of 32 or above 128, filters beyond LDS, 7x7
    stride 2) run on the generic implicit-GEMM kernel.  i8 is bit-exact; f16 /
    bf16 within the Frobenius bar."""
    rng = np.random.default_rng(7)
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=_DT[dt], pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    x, f = _conv_inputs(rng, dt, n, h, w, cin, cout, kh, kw)
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda,
                  case=f"generic conv {dt} {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{stride} d{dil}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    if dt == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= MM_FROB


def _conv_text(src, filt, out, res, grid, coords, out_coords, pad, stride, dil, et, rt):
    """A load_conv2d program in xt text (the DSL fixes the batch tile at 1, the
    result at all filter channels and f32)."""
    s = "x".join(map(str, src))
    f = "x".join(map(str, filt))
    o = "x".join(map(str, out))
    r = "x".join(map(str, res))
    g = ", ".join(map(str, grid))
    return f"""
func.func @conv(%src: memref<{s}x{et}>, %filt: memref<{f}x{et}>, %out: memref<{o}x{rt}>) attributes {{xt.grid = array<i32: {g}>}} {{
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %c0 = arith.constant 0 : i32
  %c1 = arith.constant 1 : i32
  %w = xt.load(%filt, %c0, %c0, %c0, %c0) {{shared = 2 : i64}} : (memref<{f}x{et}>, i32, i32, i32, i32) -> tensor<{f}x{et}>
  %t = xt.load_conv2d(%src, %w, {coords}) {{dilation = array<i64: {dil[0]}, {dil[1]}>, group = 1 : i64, pad = array<i64: {pad[0]}, {pad[1]}, {pad[2]}, {pad[3]}>, stride = array<i64: {stride[0]}, {stride[1]}>}} : (memref<{s}x{et}>, tensor<{f}x{et}>, i32, i32, i32, i32) -> tensor<{r}x{rt}>
  xt.store(%t, %out, {out_coords}) : (tensor<{r}x{rt}>, memref<{o}x{rt}>, i32, i32, i32, i32) -> ()
  func.return
}}"""


@pytest.mark.parametrize("et", ["i8", "bf16"])
@pytest.mark.parametrize("rt", ["f32", "bf16"])
def test_conv2d_batch_tile_channel_subset_and_bf16_result(cuda, et, rt):
    """Forms the verifier allows beyond the DSL's (lib/xt/XTOps.cpp:43-90): a
    batch tile of 2, a result holding the first 32 of the filter's 48 output
    channels, a bf16 result, a constant tile-row coordinate (row tile 1) and a
    permuted grid (bid#2 = batch, bid#0 = column tile)."""
    rng = np.random.default_rng(8)
    src, filt = (4, 12, 16, 32), (3, 3, 32, 48)
    res, out = (2, 4, 8, 32), (4, 12, 16, 32)
    mod = xt.parse(_conv_text(src, filt, out, res, (2, 1, 2), "%bid#2, %c1, %bid#0, %c0",
                              "%bid#2, %c1, %bid#0, %c0", (1, 1, 1, 1), (1, 1), (1, 1), et, rt))
    x, f = _conv_inputs(rng, et, 4, 12, 16, 32, 48, 3, 3)
    o = np.zeros(out, np.float32 if rt == "f32" else np.uint16)
    got = run_gpu(mod, [x, f, o], [et, et, rt], cuda, case=f"conv tile 2x4x8x32 of 48 {et}->{rt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    if rt == "bf16":
        got, want = bf16_bits_to_f32(got), bf16_bits_to_f32(want)
    # rows 4..7 of every image hold the result, the rest stays zero
    assert not np.any(want[:, :4]) and not np.any(want[:, 8:]) and np.any(want[:, 4:8])
    if et == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize("et", ["i8", "bf16"])
def test_conv2d_batch_tiles_covering_the_output(cuda, et):
    """Blocks of 2 images x the whole image x every output channel cover the
    output: the implicit-GEMM kernel takes them (the band kernel wants one
    image per Block)."""
    rng = np.random.default_rng(17)
    src, filt = (4, 12, 16, 32), (3, 3, 32, 64)
    res, out = (2, 12, 16, 64), (4, 12, 16, 64)
    mod = xt.parse(_conv_text(src, filt, out, res, (2, 1, 1), "%bid#0, %c0, %c0, %c0", "%bid#0, %c0, %c0, %c0",
                              (1, 1, 1, 1), (1, 1), (1, 1), et, "f32"))
    x, f = _conv_inputs(rng, et, 4, 12, 16, 32, 64, 3, 3)
    o = np.zeros(out, np.float32)
    got = run_gpu(mod, [x, f, o], [et, et, "f32"], cuda, case=f"conv batch tiles of 2 {et}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    if et == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= MM_FROB


# -- matmul epilogue and i8 (kernels/matmul.py) ---------------------------------


def _i8_inputs(rng, m, n, k):
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    # scale so that roughly a fifth of the outputs saturate and the rest spread over i8
    s = (rng.uniform(0.5, 2.0, (1, n)) / (np.sqrt(k) * 64)).astype(np.float32)
    bias = rng.uniform(-20, 20, (1, n)).astype(np.float32)
    return a, b, s, bias


@pytest.mark.parametrize(
    "m_,n_,k_,tm,tn",
    [(128, 128, 256, 64, 64), (512, 512, 1024, 64, 64), (256, 384, 512, 64, 64), (256, 256, 4096, 64, 64),
     (192, 128, 128, 64, 64)],
)
def test_matmul_i8_epilogue_bit_exact(cuda, m_, n_, k_, tm, tn):
    """The reference program kernels/matmul.py: i8 x i8 -> f32, * scale + bias,
    astype(int8).  Exact i32 accumulation, f32 conversion, two f32 roundings and
    ftoi (half to even, saturating) make the result bit-exact.  K = 4096 pushes
    |acc| past 2^24, so the int -> f32 rounding is exercised."""
    rng = np.random.default_rng(6)
    mod = K.matmul_i8(m_, n_, k_, tm, tn)
    a, b, s, bias = _i8_inputs(rng, m_, n_, k_)
    c = np.zeros((m_, n_), np.int8)
    got = run_gpu(mod, [a, b, c, s, bias], ["i8", "i8", "i8", "f32", "f32"], cuda,
                  case=f"mm i8 {m_}x{n_}x{k_} tile {tm}x{tn}")[2]
    want = run_oracle(mod, [a, b, c, s, bias], oracle_threads())[2]
    assert np.array_equal(got, want)
    assert 0.05 < np.mean((want == 127) | (want == -128)) < 0.5


def _matmul_epilogue_program(m, n, k, dt_in, scale, bias, ftoi):
    """store([ftoi]((matmul [* s]) [+ b])) with full-K 64x64 Blocks."""
    from xtile_amd import Array, bid, cdiv, convert, float32, int8, kernel, load, matmul, store, astype

    @kernel
    def prog(lhs, rhs, res, sc, bi, tm, tn, tk):
        x = bid(0)
        y = bid(1)
        t = matmul(load(lhs, index=(x, 0), shape=(tm, tk)), load(rhs, index=(0, y), shape=(tk, tn), shared=1))
        if scale:
            t = t * load(sc, index=(0, y), shape=(1, tn), shared=1)
        if bias:
            t = t + load(bi, index=(0, y), shape=(1, tn), shared=1)
        if ftoi:
            t = astype(t, dtype=int8)
        store(res, index=(x, y), tile=t)

    args = (Array(shape=(m, k), dtype=dt_in), Array(shape=(k, n), dtype=dt_in),
            Array(shape=(m, n), dtype=int8 if ftoi else float32), Array(shape=(1, n), dtype=float32),
            Array(shape=(1, n), dtype=float32), 64, 64, k)
    return convert(prog, args=args, grid=(cdiv(m, 64), cdiv(n, 64), 1))


@pytest.mark.parametrize(
    "dt,scale,bias,ftoi",
    [("i8", False, False, False), ("i8", True, False, False), ("i8", False, True, True),
     ("f16", True, True, False), ("bf16", True, True, False), ("f16", False, True, True)],
)
def test_matmul_epilogue_variants(cuda, dt, scale, bias, ftoi):
    """Every part of the epilogue is optional; f16/bf16 tiles take it too."""
    rng = np.random.default_rng(7)
    m_, n_, k_ = 256, 256, 512
    dt_in = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}[dt]
    mod = _matmul_epilogue_program(m_, n_, k_, dt_in, scale, bias, ftoi)
    if dt == "i8":
        a, b, s, bi = _i8_inputs(rng, m_, n_, k_)
    else:
        a = rng.normal(0, 1, (m_, k_)).astype(np.float32)
        b = rng.normal(0, 1, (k_, n_)).astype(np.float32)
        a, b = (f32_to_bf16_bits(a), f32_to_bf16_bits(b)) if dt == "bf16" else (a.astype(np.float16), b.astype(np.float16))
        s = rng.uniform(0.05, 0.2, (1, n_)).astype(np.float32)
        bi = rng.uniform(-3, 3, (1, n_)).astype(np.float32)
    c = np.zeros((m_, n_), np.int8 if ftoi else np.float32)
    dts = [dt, dt, "i8" if ftoi else "f32", "f32", "f32"]
    got = run_gpu(mod, [a, b, c, s, bi], dts, cuda, case=f"mm epilogue {dt} s={scale} b={bias} ftoi={ftoi}")[2]
    want = run_oracle(mod, [a, b, c, s, bi], oracle_threads())[2]
    if dt == "i8":
        assert np.array_equal(got, want)  # exact accumulation: bit-exact in every variant
    elif ftoi:
        # f32 accumulation order differs from the oracle's double sums: allow
        # the rare flip at a rounding boundary
        assert np.mean(got != want) < 1e-3 and np.max(np.abs(got.astype(int) - want.astype(int))) <= 1
    else:
        assert frob_rel(got, want) <= MM_FROB


@pytest.mark.parametrize(
    "dt,m_,n_,k_",
    [("f16", 1024, 1024, 4096),   # 64 tiles of 128 x 128: K in 4 ranges of 32 stages
     ("bf16", 1024, 2048, 2048),  # 128 tiles: 2 ranges
     ("f16", 512, 768, 1536),     # 24 tiles: K 1536 = 48 stages, 3 ranges
     ("f16", 256, 256, 9280),     # 4 tiles: 290 stages in 18 ranges of 16-17 (even spread)
     ("bf16", 256, 256, 8768)],   # 274 stages in 17 ranges of 16-17
)
def test_matmul_k_split(cuda, dt, m_, n_, k_):
    """f32 GEMMs without an epilogue whose 256 x 256 tiles would fill at most
    an eighth of the CUs run 128 x 128 tiles and split K; the partial sums are added atomically into the
    zero-filled output (the output starts non-zero here, so the fill is
    checked too)."""
    rng = np.random.default_rng(14)
    mod = K.matmul_bf16(m_, n_, k_, 256, 128) if dt == "bf16" else K.matmul_f16(m_, n_, k_, 128, 128)
    a = rng.normal(0, 1, (m_, k_)).astype(np.float32)
    b = rng.normal(0, 1, (k_, n_)).astype(np.float32)
    a, b = (f32_to_bf16_bits(a), f32_to_bf16_bits(b)) if dt == "bf16" else (a.astype(np.float16), b.astype(np.float16))
    c = np.full((m_, n_), 5.0, np.float32)
    got = run_gpu(mod, [a, b, c], [dt, dt, "f32"], cuda, case=f"mm k-split {dt} {m_}x{n_}x{k_}")[2]
    want = run_oracle(mod, [a, b, np.zeros_like(c)], oracle_threads())[2]
    assert frob_rel(got, want) <= MM_FROB


def test_k_split_opt_out_is_reproducible(cuda, monkeypatch):
    """XTILE_AMD_KSPLIT=0 keeps the tiles of a GEMM and of an implicit-GEMM
    conv that would split K whole: no atomic partial sums, so repeated
    launches give the same bits, within the bar of the oracle."""
    import torch

    monkeypatch.setenv("XTILE_AMD_KSPLIT", "0")
    rng = np.random.default_rng(15)
    dev = torch.device("cuda:0")
    m_, n_, k_ = 1024, 1024, 4096  # 64 tiles of 128 x 128: split in 4 unless opted out
    mod = K.matmul_f16(m_, n_, k_, 128, 128)
    a = rng.normal(0, 1, (m_, k_)).astype(np.float16)
    b = rng.normal(0, 1, (k_, n_)).astype(np.float16)
    bufs = [torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), torch.zeros((m_, n_), device=dev)]
    outs = []
    for i in range(3):
        print(f"[gpu] mm k-split opted out, launch {i}", flush=True)
        bufs[2].fill_(7.0)
        xt.launch(mod, *bufs)
        torch.cuda.synchronize()
        outs.append(bufs[2].cpu().numpy())
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs)
    want = run_oracle(mod, [a, b, np.zeros((m_, n_), np.float32)], oracle_threads())[2]
    assert frob_rel(outs[0], want) <= MM_FROB
    # a conv whose 52 tiles would split K in 4
    mod = K.conv2d(32, 7, 7, 512, 512, 3, 3, 7, 7)
    x = rng.normal(0, 0.1, (32, 7, 7, 512)).astype(np.float16)
    f = rng.normal(0, 0.1, (3, 3, 512, 512)).astype(np.float16)
    bufs = [torch.from_numpy(x).to(dev), torch.from_numpy(f).to(dev), torch.zeros((32, 7, 7, 512), device=dev)]
    outs = []
    for i in range(3):
        print(f"[gpu] conv igemm k-split opted out, launch {i}", flush=True)
        bufs[2].fill_(7.0)
        xt.launch(mod, *bufs)
        torch.cuda.synchronize()
        outs.append(bufs[2].cpu().numpy())
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs)
    want = run_oracle(mod, [x, f, np.zeros((32, 7, 7, 512), np.float32)], oracle_threads())[2]
    assert frob_rel(outs[0], want) <= MM_FROB


@pytest.mark.parametrize(
    "dt,m_,n_,k_,scale,bias,ftoi",
    [("f16", 4096, 2176, 256, False, False, False),   # 16 x 17 = 272 tiles of 256 x 128
     ("bf16", 4096, 2176, 384, True, True, False),
     ("i8", 4096, 2176, 512, True, True, True),        # i8 B rows of 128 bytes
     ("f16", 2176, 4096, 256, False, True, False),    # 17 x 16 = 272 tiles of 128 x 256
     ("i8", 2176, 4096, 256, False, False, False),
     ("i8", 640, 1152, 512, True, False, True)],      # 5 x 9 = 45 tiles of 128 x 128
)
def test_matmul_rectangular_dma_tiles(cuda, dt, m_, n_, k_, scale, bias, ftoi):
    """GEMMs whose Blocks do not map onto 256 x 256 tiles (M or N an odd
    multiple of 128) run the DMA kernel at 256 x 128, 128 x 256 or 128 x 128,
    with every epilogue form and i8 results."""
    rng = np.random.default_rng(16)
    dt_in = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}[dt]
    mod = _matmul_epilogue_program(m_, n_, k_, dt_in, scale, bias, ftoi)
    if dt == "i8":
        a, b, s, bi = _i8_inputs(rng, m_, n_, k_)
    else:
        a = rng.normal(0, 1, (m_, k_)).astype(np.float32)
        b = rng.normal(0, 1, (k_, n_)).astype(np.float32)
        a, b = (f32_to_bf16_bits(a), f32_to_bf16_bits(b)) if dt == "bf16" else (a.astype(np.float16), b.astype(np.float16))
        s = rng.uniform(0.05, 0.2, (1, n_)).astype(np.float32)
        bi = rng.uniform(-3, 3, (1, n_)).astype(np.float32)
    c = np.zeros((m_, n_), np.int8 if ftoi else np.float32)
    dts = [dt, dt, "i8" if ftoi else "f32", "f32", "f32"]
    got = run_gpu(mod, [a, b, c, s, bi], dts, cuda, case=f"mm rect {dt} {m_}x{n_}x{k_} s={scale} b={bias} ftoi={ftoi}")[2]
    want = run_oracle(mod, [a, b, c, s, bi], oracle_threads())[2]
    if dt == "i8":
        assert np.array_equal(got, want)
    elif ftoi:
        assert np.mean(got != want) < 1e-3 and np.max(np.abs(got.astype(int) - want.astype(int))) <= 1
    else:
        assert frob_rel(got, want) <= MM_FROB


def test_matmul_k_split_in_a_graph(cuda):
    """A K-split GEMM (zero-fill kernel, then atomic partial sums) captured in
    a HIP graph and replayed three times with eager work between: every replay
    matches the eager launch to a relative 1e-6 (the addition order varies)."""
    import torch

    rng = np.random.default_rng(15)
    m_, n_, k_ = 1024, 1024, 4096
    mod = K.matmul_f16(m_, n_, k_, 128, 128)
    a = rng.normal(0, 1, (m_, k_)).astype(np.float16)
    b = rng.normal(0, 1, (k_, n_)).astype(np.float16)
    eager = run_gpu(mod, [a, b, np.zeros((m_, n_), np.float32)], ["f16", "f16", "f32"], cuda, case="mm k-split eager")[2]
    print("[gpu] mm k-split graph capture", flush=True)
    da, db = torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)
    dc = torch.zeros(m_, n_, dtype=torch.float32, device=cuda)
    stream = torch.cuda.Stream(device=cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        xt.launch(mod, da, db, dc, stream=stream)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            xt.launch(mod, da, db, dc, stream=stream)
    torch.cuda.synchronize()
    for r in range(3):
        dc.fill_(float(r - 7))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert frob_rel(dc.cpu().numpy(), eager) <= 1e-6, r


def test_reference_traced_matmul_program(cuda):
    """tests/golden/dsl/matmul_int8_epilogue.mlir is the text the reference's own
    tracer (xtile/dsl.py) wrote for the kernels/matmul.py program: parsed as-is
    and run on the GPU, bit-exact against the oracle."""
    from pathlib import Path

    text = (Path(__file__).parent / "golden" / "dsl" / "matmul_int8_epilogue.mlir").read_text()
    mod = xt.parse(text)
    sig = xt.signature(mod)
    shapes = [tuple(a["shape"]) for a in sig["args"]]
    assert shapes == [(1024, 256), (256, 512), (1024, 512), (1, 512), (1, 512)]
    rng = np.random.default_rng(8)
    a, b, s, bias = _i8_inputs(rng, 1024, 512, 256)
    c = np.zeros((1024, 512), np.int8)
    got = run_gpu(mod, [a, b, c, s, bias], ["i8", "i8", "i8", "f32", "f32"], cuda, case="reference-traced matmul")[2]
    want = run_oracle(mod, [a, b, c, s, bias], oracle_threads())[2]
    assert np.array_equal(got, want)


@pytest.mark.parametrize(
    "n,h,w,cin,cout,kh,kw,th,tw,pad,stride,dil,dt",
    [
        (1, 64, 64, 3, 64, 7, 7, 8, 32, (3, 3, 3, 3), (2, 2), (1, 1), "f16"),   # the RGB stem
        (2, 30, 40, 3, 64, 7, 7, 5, 20, (3, 3, 3, 3), (2, 2), (1, 1), "bf16"),
        (2, 20, 150, 3, 24, 3, 3, 4, 150, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),  # 2 pixel chunks, Cout 24
        (1, 17, 33, 1, 8, 5, 5, 13, 17, (2, 1, 2, 3), (1, 2), (2, 1), "f16"),   # Cin 1, row dilation
        (3, 10, 12, 5, 136, 3, 3, 5, 12, (1, 1, 1, 1), (1, 1), (1, 1), "f16"),  # Cout tile past 128
        (2, 31, 29, 6, 72, 3, 3, 15, 29, (0, 1, 1, 1), (2, 1), (1, 1), "bf16"),
        (1, 40, 300, 4, 32, 1, 1, 8, 300, (0, 0, 0, 0), (1, 1), (1, 1), "f16"),  # 1 x 1, 3 chunks
        (1, 64, 64, 3, 64, 7, 7, 8, 32, (3, 3, 3, 3), (2, 2), (1, 1), "i8"),
        (2, 20, 150, 5, 48, 3, 3, 4, 150, (1, 1, 1, 1), (1, 1), (1, 1), "i8"),
        (1, 17, 33, 12, 16, 5, 5, 13, 17, (2, 1, 2, 3), (1, 2), (2, 1), "i8"),
        (1, 30, 40, 15, 32, 7, 7, 5, 20, (3, 3, 3, 3), (2, 2), (1, 1), "i8"),   # one staging round
        (2, 33, 47, 12, 64, 3, 3, 17, 12, (1, 1, 1, 1), (2, 2), (1, 1), "f16"),  # Cin past 8: wider patch rows
        (2, 33, 47, 12, 64, 3, 3, 17, 12, (1, 1, 1, 1), (2, 2), (1, 1), "bf16"),
        (1, 29, 35, 20, 32, 3, 3, 5, 18, (1, 1, 1, 1), (2, 2), (1, 1), "f16"),
        (1, 29, 35, 20, 32, 3, 3, 5, 18, (1, 1, 1, 1), (2, 2), (1, 1), "bf16"),
        (1, 24, 30, 13, 48, 5, 5, 6, 15, (2, 2, 2, 2), (1, 1), (1, 1), "f16"),   # odd Cin, 5 x 5
        # >= 2048 output-row chunks with one channel tile: workgroups walk the chunks
        (32, 224, 224, 3, 64, 7, 7, 4, 112, (3, 3, 3, 3), (2, 2), (1, 1), "f16"),  # C8's stem, 3584 chunks
        (32, 128, 128, 3, 64, 7, 7, 4, 64, (3, 3, 3, 3), (2, 2), (1, 1), "bf16"),  # 2048 chunks
        (32, 128, 128, 3, 32, 7, 7, 4, 64, (3, 3, 3, 3), (2, 2), (1, 1), "i8"),    # Cout 32: half a channel tile
        (67, 62, 62, 3, 64, 7, 7, 1, 31, (3, 3, 3, 3), (2, 2), (1, 1), "f16"),     # 2077 chunks: uneven XCD ranges
        (40, 64, 64, 3, 16, 3, 3, 8, 64, (1, 1, 1, 1), (1, 1), (1, 1), "bf16"),    # two pieces a patch row
    ],
)
def test_conv2d_few_input_channels(cuda, n, h, w, cin, cout, kh, kw, th, tw, pad, stride, dil, dt):
    """Cin * esize not a multiple of 16 (the RGB stem; f16 / bf16 within the
    matmul bar, i8 bit-exact) with the Blocks covering the output take the
    LDS-patch kernel (conv_small.hip): the
    KH input rows of 128 output pixels staged in LDS, K in runs of KW * Cin
    rounded up to 16 with zero filter rows, pixels past the row and channels
    past Cout not stored; with one channel tile and at least 2048 row chunks
    the workgroups walk the chunks (filter staged once, the next chunk's
    patch loads in flight)."""
    rng = np.random.default_rng(21)
    xdt = {"bf16": xt.bfloat16, "f16": xt.float16, "i8": xt.int8}[dt]
    mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xdt, pad=pad, stride=stride, dilation=dil)
    oh = (h + pad[0] + pad[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    if dt == "i8":
        x = rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8)
        f = rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8)
    else:
        x = rng.normal(0, 0.5, (n, h, w, cin)).astype(np.float32)
        f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
        if dt == "bf16":
            x, f = f32_to_bf16_bits(x), f32_to_bf16_bits(f)
        else:
            x, f = x.astype(np.float16), f.astype(np.float16)
    o = np.zeros((n, oh, ow, cout), np.float32)
    got = run_gpu(mod, [x, f, o], [dt, dt, "f32"], cuda,
                  case=f"conv few channels {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{stride} d{dil} {dt}")[2]
    want = run_oracle(mod, [x, f, o], oracle_threads())[2]
    if dt == "i8":  # exact i32 sums rounded to f32 once
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= MM_FROB
