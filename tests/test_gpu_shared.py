"""GPU parity of the shared=k leader rule where it changes the result.

A load with `shared = k` is evaluated once per sharing group: the reference's
xt-serialize keeps the first Block's tile in z -> y -> x order
(lib/xt/XTSerialize.cpp:86-101; test/xt/serialize.mlir:55-136), which is the
load evaluated with bid_i = 0 for every axis i < k.  In every program below
the shared load's coordinates move along an axis < k, and the memref is large
enough that every Block's own tile is in range and holds different values, so
a kernel that ignored the rule (or forced one axis too many) would read other
tiles.  Each case runs through one kernel family (ew_binary, gemm including
the fused-Block and i8-epilogue forms, conv2d, the fused generator and the
tile interpreter) and is compared with the C oracle (closed form: leader
coordinates) and with oracle/interp.py (literal serialize).  The same oracle
run on the program with the rule planted wrong (shared removed, or one axis
too many) must differ from the GPU result, so each case can tell the rules
apart.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from oracle import f32_to_bf16_bits, interp
from tests.gpu_util import frob_rel, run_gpu, run_oracle

pytestmark = pytest.mark.gpu

MM_FROB = 1e-3


def _program(sig: str, grid, body: str) -> str:
    return (
        f"func.func @k({sig}) attributes {{xt.grid = array<i32: {grid[0]}, {grid[1]}, {grid[2]}>}} {{\n"
        "  %bid:3 = xt.get_tile_block_id : i32, i32, i32\n"
        "  %zero = arith.constant 0 : i32\n"
        f"{body}\n"
        "  func.return\n}"
    )


def _interp(text, host):
    bufs = [np.array(h, copy=True) for h in host]
    interp.run(text, bufs)
    return bufs


def _close(kind: str, got, want) -> bool:
    if kind == "exact":
        return np.array_equal(np.asarray(got).view(np.uint8), np.asarray(want).view(np.uint8))
    if kind == "frob":
        return frob_rel(got, want) <= MM_FROB
    return np.allclose(got, want, rtol=2e-5, atol=1e-6)


def _check(cuda, text, host, dtypes, out, kind, kernel, planted, case):
    """GPU == C oracle == literal serialize; every planted rule differs."""
    m = xt.parse(text)
    assert xt.plan(m)["kernel"].startswith(kernel), xt.plan(m)["kernel"]
    got = run_gpu(m, host, dtypes, cuda, case=case)[out]
    want = run_oracle(m, host, 4)[out]
    literal = _interp(text, host)[out]
    assert _close(kind, want, literal), "oracle closed form and literal serialize disagree"
    assert _close(kind, got, want), f"{case}: GPU result differs from the oracle"
    for wrong_text in planted:
        wrong = run_oracle(xt.parse(wrong_text), host, 4)[out]
        assert not _close(kind, got, wrong), f"{case}: a planted sharing rule gives the same result"


def _plants(text: str, k: int):
    """The rule planted wrong: sharing dropped, and (k < 2) one more axis forced."""
    out = [text.replace(f" {{shared = {k} : i64}}", "")]
    if k < 2:
        out.append(text.replace(f"{{shared = {k} : i64}}", f"{{shared = {k + 1} : i64}}"))
    return out


# -- ew_binary -----------------------------------------------------------------------


@pytest.mark.parametrize("k", [1, 2])
def test_ew_binary_shared_moving_index(cuda, k):
    """c[x, y] = a[leader tile] + b[x, y]; a's tile index is (bid0, bid1)."""
    t = "tensor<32x64xf32>"
    mr = "memref<128x256xf32>"
    body = (
        f"  %0 = xt.load(%a, %bid#0, %bid#1) {{shared = {k} : i64}} : ({mr}, i32, i32) -> {t}\n"
        f"  %1 = xt.load(%b, %bid#0, %bid#1) : ({mr}, i32, i32) -> {t}\n"
        f"  %2 = xt.add(%0, %1) : {t}, {t} -> {t}\n"
        f"  xt.store(%2, %c, %bid#0, %bid#1) : ({t}, {mr}, i32, i32) -> ()"
    )
    text = _program(f"%a: {mr}, %b: {mr}, %c: {mr}", (4, 4, 1), body)
    rng = np.random.default_rng(10 + k)
    a = rng.uniform(-1, 1, (128, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, (128, 256)).astype(np.float32)
    host = [a, b, np.zeros_like(a)]
    _check(cuda, text, host, ["f32"] * 3, 2, "exact", "ew_binary", _plants(text, k), f"ew shared={k}")
    got = run_gpu(xt.parse(text), host, ["f32"] * 3, cuda, case=f"ew shared={k} closed form")[2]
    lead = np.tile(a[:32, :64] if k == 2 else a[:32, :], (4, 4 if k == 2 else 1))
    assert np.array_equal(got, lead + b)


# -- gemm --------------------------------------------------------------------------------


def _mm_text(elem, M, N, K, tm, tn, grid, a_idx, b_idx, a_rows_mul, b_rows_mul, a_shared, b_shared,
             out_elem="f32"):
    am = f"memref<{M * a_rows_mul[0]}x{K * a_rows_mul[1]}x{elem}>"
    bm = f"memref<{K * b_rows_mul[0]}x{N * b_rows_mul[1]}x{elem}>"
    cm = f"memref<{M}x{N}x{out_elem}>"
    at, bt, ct = f"tensor<{tm}x{K}x{elem}>", f"tensor<{K}x{tn}x{elem}>", f"tensor<{tm}x{tn}xf32>"
    sa = f" {{shared = {a_shared} : i64}}" if a_shared else ""
    sb = f" {{shared = {b_shared} : i64}}" if b_shared else ""
    body = (
        f"  %x = xt.load(%a, {a_idx}){sa} : ({am}, i32, i32) -> {at}\n"
        f"  %x2 = xt.load(%b, {b_idx}){sb} : ({bm}, i32, i32) -> {bt}\n"
        f"  %m = xt.matmul(%x, %x2) : {at}, {bt} -> {ct}\n"
        f"  xt.store(%m, %c, %bid#0, %bid#1) : ({ct}, {cm}, i32, i32) -> ()"
    )
    return _program(f"%a: {am}, %b: {bm}, %c: {cm}", grid, body), am, bm


@pytest.mark.parametrize(
    "case,elem,tm,tn,k",
    [
        ("B moves along axis 0, 128x128 Blocks", "f16", 128, 128, 1),
        ("B moves along the fused axis, 64x64 Blocks", "f16", 64, 64, 1),
        ("B moves along axes 0 and 1", "bf16", 128, 128, 2),
    ],
)
def test_gemm_shared_b_moving_index(cuda, case, elem, tm, tn, k):
    """B's tile index is (bid0, bid1) with shared=k: every Block multiplies by
    the leader's B rows.  With 64x64 Blocks the kernel fuses four Blocks along
    axis 0 into one 256-row workgroup tile, whose B panel must be the leader's."""
    M, N, K = 512, 512, 256
    grid = (M // tm, N // tn, 1)
    b_idx = "%bid#0, %bid#1"
    text, am, bm = _mm_text(elem, M, N, K, tm, tn, grid, "%bid#0, %zero", b_idx, (1, 1), (grid[0], 1), 0, k)
    rng = np.random.default_rng(20 + tm + k)
    if elem == "f16":
        a = rng.uniform(-1, 1, (M, K)).astype(np.float16)
        b = rng.uniform(-1, 1, (K * grid[0], N)).astype(np.float16)
    else:
        a = f32_to_bf16_bits(rng.normal(0, 0.5, (M, K)).astype(np.float32))
        b = f32_to_bf16_bits(rng.normal(0, 0.5, (K * grid[0], N)).astype(np.float32))
    host = [a, b, np.zeros((M, N), np.float32)]
    _check(cuda, text, host, [elem, elem, "f32"], 2, "frob", "gemm", _plants(text, k), f"gemm {case}")


def test_gemm_shared_a_moving_index(cuda):
    """C5's form (A shared=1, C stored at (bid1, bid0)) with A's index (bid1, bid0):
    every Block uses the leader's K columns of A."""
    M, N, K, tm, tn = 512, 1024, 256, 256, 128
    grid = (N // tn, M // tm, 1)
    am = f"memref<{M}x{K * grid[0]}xbf16>"
    bm = f"memref<{K}x{N}xbf16>"
    cm = f"memref<{M}x{N}xf32>"
    at, bt, ct = f"tensor<{tm}x{K}xbf16>", f"tensor<{K}x{tn}xbf16>", f"tensor<{tm}x{tn}xf32>"
    body = (
        f"  %x = xt.load(%a, %bid#1, %bid#0) {{shared = 1 : i64}} : ({am}, i32, i32) -> {at}\n"
        f"  %x2 = xt.load(%b, %zero, %bid#0) : ({bm}, i32, i32) -> {bt}\n"
        f"  %m = xt.matmul(%x, %x2) : {at}, {bt} -> {ct}\n"
        f"  xt.store(%m, %c, %bid#1, %bid#0) : ({ct}, {cm}, i32, i32) -> ()"
    )
    text = _program(f"%a: {am}, %b: {bm}, %c: {cm}", grid, body)
    rng = np.random.default_rng(31)
    a = f32_to_bf16_bits(rng.normal(0, 0.5, (M, K * grid[0])).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.5, (K, N)).astype(np.float32))
    host = [a, b, np.zeros((M, N), np.float32)]
    _check(cuda, text, host, ["bf16", "bf16", "f32"], 2, "frob", "gemm", _plants(text, 1), "gemm A shared=1")


def test_gemm_i8_epilogue_shared_moving_index(cuda):
    """kernels/matmul.py's i8 form with 64x64 Blocks (fused into larger
    workgroup tiles) where B, scale and bias all take a shared=1 index that
    moves along axis 0: the leader's rows of each."""
    M, N, K, t = 512, 512, 256, 64
    g = M // t
    am, bm, cm = f"memref<{M}x{K}xi8>", f"memref<{K * g}x{N}xi8>", f"memref<{M}x{N}xi8>"
    vm = f"memref<{g}x{N}xf32>"
    at, bt, ct, vt = f"tensor<{t}x{K}xi8>", f"tensor<{K}x{t}xi8>", f"tensor<{t}x{t}xf32>", f"tensor<1x{t}xf32>"
    body = (
        f"  %x = xt.load(%a, %bid#0, %zero) : ({am}, i32, i32) -> {at}\n"
        f"  %x2 = xt.load(%b, %bid#0, %bid#1) {{shared = 1 : i64}} : ({bm}, i32, i32) -> {bt}\n"
        f"  %x3 = xt.load(%s, %bid#0, %bid#1) {{shared = 1 : i64}} : ({vm}, i32, i32) -> {vt}\n"
        f"  %x4 = xt.load(%bias, %bid#0, %bid#1) {{shared = 1 : i64}} : ({vm}, i32, i32) -> {vt}\n"
        f"  %m = xt.matmul(%x, %x2) : {at}, {bt} -> {ct}\n"
        f"  %n = xt.mul(%m, %x3) : {ct}, {vt} -> {ct}\n"
        f"  %o = xt.add(%n, %x4) : {ct}, {vt} -> {ct}\n"
        f"  %q = xt.ftoi(%o) : {ct} -> tensor<{t}x{t}xi8>\n"
        f"  xt.store(%q, %c, %bid#0, %bid#1) : (tensor<{t}x{t}xi8>, {cm}, i32, i32) -> ()"
    )
    text = _program(f"%a: {am}, %b: {bm}, %c: {cm}, %s: {vm}, %bias: {vm}", (g, N // t, 1), body)
    rng = np.random.default_rng(41)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    b = rng.integers(-128, 128, (K * g, N), dtype=np.int8)
    s = (rng.uniform(0.5, 2.0, (g, N)) / (np.sqrt(K) * 64)).astype(np.float32)
    bias = rng.uniform(-20, 20, (g, N)).astype(np.float32)
    host = [a, b, np.zeros((M, N), np.int8), s, bias]
    _check(cuda, text, host, ["i8", "i8", "i8", "f32", "f32"], 2, "exact", "gemm i8", _plants(text, 1),
           "gemm i8 epilogue shared=1")


# -- conv2d ------------------------------------------------------------------------------


@pytest.mark.parametrize("k,axis,tile_h", [(2, 0, 4), (2, 1, 4), (1, 0, 4), (1, 1, 4), (2, 1, 2)])
def test_conv_shared_filter_moving_index(cuda, k, axis, tile_h):
    """The filter is loaded at (bid_axis, 0, 0, 0) from a stack of filters
    along KH with shared=k.  Grid axis 0 walks the batch and axis 1 the row
    tiles.  For axis < k every Block convolves with the leader's filter
    (filter 0); for k=1 on axis 1 the filter moves with the row tile and no
    sharing applies, so each Block uses its own."""
    N, H, W, CI, CO = 2, 8, 8, 32, 64
    grid = (N, H // tile_h, 1)
    nf = grid[axis]
    fm = f"memref<{3 * nf}x3x{CI}x{CO}xf16>"
    sm, om = f"memref<{N}x{H}x{W}x{CI}xf16>", f"memref<{N}x{H}x{W}x{CO}xf32>"
    ft, rt = f"tensor<3x3x{CI}x{CO}xf16>", f"tensor<1x{tile_h}x{W}x{CO}xf32>"
    body = (
        f"  %f = xt.load(%filt, %bid#{axis}, %zero, %zero, %zero) {{shared = {k} : i64}} : ({fm}, i32, i32, i32, i32) -> {ft}\n"
        f"  %y = xt.load_conv2d(%src, %f, %bid#0, %bid#1, %zero, %zero) {{dilation = array<i64: 1, 1>, group = 1 : i64, "
        f"pad = array<i64: 1, 1, 1, 1>, stride = array<i64: 1, 1>}} : ({sm}, {ft}, i32, i32, i32, i32) -> {rt}\n"
        f"  xt.store(%y, %out, %bid#0, %bid#1, %zero, %zero) : ({rt}, {om}, i32, i32, i32, i32) -> ()"
    )
    text = _program(f"%src: {sm}, %filt: {fm}, %out: {om}", grid, body)
    rng = np.random.default_rng(50 + 10 * k + axis + tile_h)
    x = rng.normal(0, 0.5, (N, H, W, CI)).astype(np.float16)
    f = rng.normal(0, 0.5, (3 * nf, 3, CI, CO)).astype(np.float16)
    host = [x, f, np.zeros((N, H, W, CO), np.float32)]
    # the plant that moves this index: sharing dropped when the axis is
    # shared, one axis too many (k=2) when it is not
    plants = _plants(text, k)[:1] if axis < k else _plants(text, k)[1:]
    _check(cuda, text, host, ["f16", "f16", "f32"], 2, "frob", "conv2d", plants,
           f"conv shared={k} axis={axis} tile_h={tile_h}")


# -- fused kernel and tile interpreter ------------------------------------------------


@pytest.mark.parametrize("fuse", ["1", "0"])
@pytest.mark.parametrize("k", [1, 2])
def test_scale_rows_shared_moving_index(cuda, monkeypatch, fuse, k):
    """y = x * g + r with g's tile index (bid0, bid1) shared=k over a stack of
    gains: fused kernel (XTILE_AMD_FUSE unset) and tile interpreter
    (XTILE_AMD_FUSE=0)."""
    monkeypatch.setenv("XTILE_AMD_FUSE", fuse)
    R, C, tr, tc = 64, 256, 8, 64
    grid = (R // tr, C // tc, 1)
    xm, gm = f"memref<{R}x{C}xf32>", f"memref<{grid[0]}x{C}xf32>"
    xt_, gt, rt = f"tensor<{tr}x{tc}xf32>", f"tensor<1x{tc}xf32>", f"tensor<{tr}x1xf32>"
    rm = f"memref<{R}x{grid[1]}xf32>"
    body = (
        f"  %x = xt.load(%in, %bid#0, %bid#1) : ({xm}, i32, i32) -> {xt_}\n"
        f"  %g = xt.load(%gain, %bid#0, %bid#1) {{shared = {k} : i64}} : ({gm}, i32, i32) -> {gt}\n"
        f"  %r = xt.load(%rows, %bid#0, %bid#1) {{shared = {k} : i64}} : ({rm}, i32, i32) -> {rt}\n"
        f"  %p = xt.mul(%x, %g) : {xt_}, {gt} -> {xt_}\n"
        f"  %q = xt.add(%p, %r) : {xt_}, {rt} -> {xt_}\n"
        f"  xt.store(%q, %out, %bid#0, %bid#1) : ({xt_}, {xm}, i32, i32) -> ()"
    )
    text = _program(f"%in: {xm}, %gain: {gm}, %rows: {rm}, %out: {xm}", grid, body)
    rng = np.random.default_rng(60 + k)
    x = rng.normal(size=(R, C)).astype(np.float32)
    g = rng.normal(size=(grid[0], C)).astype(np.float32)
    r = rng.normal(size=(R, grid[1])).astype(np.float32)
    host = [x, g, r, np.zeros_like(x)]
    kernel = "fused" if fuse == "1" else "tile_vm"
    _check(cuda, text, host, ["f32"] * 4, 3, "exact", kernel, _plants(text, k), f"{kernel} shared={k}")


@pytest.mark.parametrize("stage", ["1", "0"])
@pytest.mark.parametrize("k", [1, 2])
def test_tile_vm_matmul_shared_moving_index(cuda, monkeypatch, stage, k):
    """An f32 matmul of 16x16 tiles whose left operand's index (bid0, bid1)
    is shared=k: on the staged kernel (f32 MFMA) and on the tile interpreter
    (XTILE_AMD_STAGE=0)."""
    monkeypatch.setenv("XTILE_AMD_STAGE", stage)
    mr = "memref<64x64xf32>"
    t = "tensor<16x16xf32>"
    body = (
        f"  %x = xt.load(%a, %bid#0, %bid#1) {{shared = {k} : i64}} : ({mr}, i32, i32) -> {t}\n"
        f"  %y = xt.load(%b, %bid#0, %bid#1) : ({mr}, i32, i32) -> {t}\n"
        f"  %m = xt.matmul(%x, %y) : {t}, {t} -> {t}\n"
        f"  xt.store(%m, %c, %bid#0, %bid#1) : ({t}, {mr}, i32, i32) -> ()"
    )
    text = _program(f"%a: {mr}, %b: {mr}, %c: {mr}", (4, 4, 1), body)
    rng = np.random.default_rng(70 + k)
    a = rng.normal(size=(64, 64)).astype(np.float32)
    b = rng.normal(size=(64, 64)).astype(np.float32)
    host = [a, b, np.zeros_like(a)]
    kernel = "staged" if stage == "1" else "tile_vm"
    _check(cuda, text, host, ["f32"] * 3, 2, "close", kernel, _plants(text, k), f"{kernel} matmul shared={k}")


def test_conv_filter_at_a_constant_index_of_a_stack(cuda):
    """The filter tile is filter 1 of a stack of three (a constant coordinate,
    no sharing): every Block uses it, at a non-zero offset into the array."""
    N, H, W, CI, CO = 2, 8, 8, 32, 64
    fm = f"memref<9x3x{CI}x{CO}xf16>"
    sm, om = f"memref<{N}x{H}x{W}x{CI}xf16>", f"memref<{N}x{H}x{W}x{CO}xf32>"
    ft, rt = f"tensor<3x3x{CI}x{CO}xf16>", f"tensor<1x4x{W}x{CO}xf32>"
    body = (
        "  %one = arith.constant 1 : i32\n"
        f"  %f = xt.load(%filt, %one, %zero, %zero, %zero) : ({fm}, i32, i32, i32, i32) -> {ft}\n"
        f"  %y = xt.load_conv2d(%src, %f, %bid#0, %bid#1, %zero, %zero) {{dilation = array<i64: 1, 1>, group = 1 : i64, "
        f"pad = array<i64: 1, 1, 1, 1>, stride = array<i64: 1, 1>}} : ({sm}, {ft}, i32, i32, i32, i32) -> {rt}\n"
        f"  xt.store(%y, %out, %bid#0, %bid#1, %zero, %zero) : ({rt}, {om}, i32, i32, i32, i32) -> ()"
    )
    text = _program(f"%src: {sm}, %filt: {fm}, %out: {om}", (N, 2, 1), body)
    rng = np.random.default_rng(58)
    x = rng.normal(0, 0.5, (N, H, W, CI)).astype(np.float16)
    f = rng.normal(0, 0.5, (9, 3, CI, CO)).astype(np.float16)
    host = [x, f, np.zeros((N, H, W, CO), np.float32)]
    wrong = text.replace("%f = xt.load(%filt, %one,", "%f = xt.load(%filt, %zero,")
    _check(cuda, text, host, ["f16", "f16", "f32"], 2, "frob", "conv2d", [wrong], "conv filter 1 of a stack")
