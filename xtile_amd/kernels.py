"""Example tile programs: the reference's kernels/*.py, written with this DSL.

Each builder returns a parsed Module for one configuration.  They reproduce
the reference programs (kernels/add.py:6-30, kernels/softmax.py:10-36,
kernels/matmul.py:6-38, kernels/conv2d.py:10-59) with
the tile sizes of the five benchmark configurations:

  C1 add      fp32 1024x1024, 32x64 tiles, grid (32, 16, 1)
  C2 softmax  fp32 8192x4096, one 1x4096 row per Block, grid (8192, 1, 1)
  C3 matmul   f16 4096^3 -> f32, 128x128 Block tiles (full K), B shared along axis 0
  C4 conv2d   f16 NHWC 32x56x56x64, 3x3x64x64 filter, stride 1, pad 1 -> f32
  C5 matmul   bf16 4096x11008x4096 -> f32, 256x128 tiles, grid (86, 16, 1),
              A shared along axis 0 (`shared = 1`)
"""

from __future__ import annotations

from . import (
    Array,
    add as tile_add,
    astype,
    bfloat16,
    bid,
    cdiv,
    convert,
    exp,
    float16,
    float32,
    int8,
    kernel,
    load,
    load_conv2d,
    matmul,
    max as tile_max,
    mul as tile_mul,
    reciprocal,
    rsqrt,
    reshape,
    store,
    sub as tile_sub,
    sum as tile_sum,
    transpose,
)


# -- add ---------------------------------------------------------------------


@kernel
def add_kernel(lhs, rhs, out, tile_h, tile_w):
    b0 = bid(0)
    b1 = bid(1)
    a = load(lhs, index=(b0, b1), shape=(tile_h, tile_w))
    b = load(rhs, index=(b0, b1), shape=(tile_h, tile_w))
    store(out, index=(b0, b1), tile=a + b)


def add(rows: int, cols: int, tile_h: int = 32, tile_w: int = 64):
    arr = Array(shape=(rows, cols), dtype=float32)
    grid = (cdiv(rows, tile_h), cdiv(cols, tile_w), 1)
    return convert(add_kernel, args=(arr, arr, arr, tile_h, tile_w), grid=grid, double_buffering=True)


@kernel
def add_rows_kernel(lhs, rhs, out, trow, col):
    """The reference's kernels/add.py program: full-width row tiles."""
    bid_x = bid(0)
    a = load(lhs, index=(bid_x, 0), shape=(trow, col))
    b = load(rhs, index=(bid_x, 0), shape=(trow, col))
    store(out, index=(bid_x, 0), tile=a + b)


def add_rows(rows: int, cols: int, trow: int = 64):
    arr = Array(shape=(rows, cols), dtype=float32)
    return convert(
        add_rows_kernel,
        args=(arr, arr, arr, trow, cols),
        grid=(cdiv(rows, trow), 1, 1),
        double_buffering=True,
    )


# -- softmax -----------------------------------------------------------------


@kernel
def softmax_kernel(inp, out, trow, col):
    bid_x = bid(0)
    x = load(inp, index=(bid_x, 0), shape=(trow, col))
    x = x - tile_max(x, axis=-1)
    x = exp(x)
    r = tile_sum(x, axis=-1)
    x = x / r
    store(out, index=(bid_x, 0), tile=x)


def softmax(rows: int, cols: int, trow: int = 1):
    arr = Array(shape=(rows, cols), dtype=float32)
    return convert(
        softmax_kernel,
        args=(arr, arr, trow, cols),
        grid=(cdiv(rows, trow), 1, 1),
        double_buffering=True,
    )


# -- matmul ------------------------------------------------------------------


@kernel
def matmul_kernel(lhs, rhs, res, tm, tn, tk):
    """A row panel per bid(0), B column panel per bid(1) shared along axis 0."""
    bid_m = bid(0)
    bid_n = bid(1)
    a = load(lhs, index=(bid_m, 0), shape=(tm, tk))
    b = load(rhs, index=(0, bid_n), shape=(tk, tn), shared=1)
    store(res, index=(bid_m, bid_n), tile=matmul(a, b))


@kernel
def matmul_nm_kernel(lhs, rhs, res, tm, tn, tk):
    """Grid (N/tn, M/tm): bid(0) walks N, so the A panel is `shared = 1`."""
    bid_n = bid(0)
    bid_m = bid(1)
    a = load(lhs, index=(bid_m, 0), shape=(tm, tk), shared=1)
    b = load(rhs, index=(0, bid_n), shape=(tk, tn))
    store(res, index=(bid_m, bid_n), tile=matmul(a, b))


def matmul_f16(m: int, n: int, k: int, tm: int = 128, tn: int = 128):
    a = Array(shape=(m, k), dtype=float16)
    b = Array(shape=(k, n), dtype=float16)
    c = Array(shape=(m, n), dtype=float32)
    return convert(
        matmul_kernel,
        args=(a, b, c, tm, tn, k),
        grid=(cdiv(m, tm), cdiv(n, tn), 1),
        double_buffering=True,
    )


def matmul_bf16(m: int, n: int, k: int, tm: int = 256, tn: int = 128):
    a = Array(shape=(m, k), dtype=bfloat16)
    b = Array(shape=(k, n), dtype=bfloat16)
    c = Array(shape=(m, n), dtype=float32)
    return convert(
        matmul_nm_kernel,
        args=(a, b, c, tm, tn, k),
        grid=(cdiv(n, tn), cdiv(m, tm), 1),
        double_buffering=True,
    )


@kernel
def matmul_i8_kernel(lhs, rhs, res, scale, bias, tm, tn, tk):
    """kernels/matmul.py:6-19: i8 x i8 -> f32, then * scale + bias per column
    and astype(int8); B, scale and bias are shared along axis 0."""
    bid_x = bid(0)
    bid_y = bid(1)
    lhs_tile = load(lhs, index=(bid_x, 0), shape=(tm, tk))
    rhs_tile = load(rhs, index=(0, bid_y), shape=(tk, tn), shared=1)
    s_tile = load(scale, index=(0, bid_y), shape=(1, tn), shared=1)
    b_tile = load(bias, index=(0, bid_y), shape=(1, tn), shared=1)
    t = matmul(lhs_tile, rhs_tile)
    t = t * s_tile + b_tile
    t = astype(t, dtype=int8)
    store(res, index=(bid_x, bid_y), tile=t)


def matmul_i8(m: int, n: int, k: int, tm: int = 64, tn: int = 64):
    """The reference's matmul program (kernels/matmul.py:22-38, 64 x 64 tiles)."""
    a = Array(shape=(m, k), dtype=int8)
    b = Array(shape=(k, n), dtype=int8)
    c = Array(shape=(m, n), dtype=int8)
    s = Array(shape=(1, n), dtype=float32)
    bias = Array(shape=(1, n), dtype=float32)
    return convert(
        matmul_i8_kernel,
        args=(a, b, c, s, bias, tm, tn, k),
        grid=(cdiv(m, tm), cdiv(n, tn), 1),
        double_buffering=True,
    )


# -- conv2d ------------------------------------------------------------------


@kernel
def conv2d_kernel(inp, filt, out, tile_h, tile_w, cin, cout, kh, kw, pt, pl, pb, pr, sh, sw, dh, dw):
    bid_n = bid(0)
    bid_h = bid(1)
    bid_w = bid(2)
    zero = 0
    f = load(filt, index=(zero, zero, zero, zero), shape=(kh, kw, cin, cout), shared=2)
    t = load_conv2d(
        inp,
        f,
        index=(bid_n, bid_h, bid_w, zero),
        shape=(1, tile_h, tile_w, cout),
        group=1,
        pad=(pt, pl, pb, pr),
        stride=(sh, sw),
        dilation=(dh, dw),
    )
    store(out, index=(bid_n, bid_h, bid_w, zero), tile=t)


def conv2d(n, h, w, cin, cout, kh=3, kw=3, tile_h=4, tile_w=56, dtype=float16, pad=None, stride=(1, 1),
           dilation=(1, 1)):
    """NHWC conv; `pad` is (top, left, bottom, right), by default "same" for odd
    filters as in kernels/conv2d.py:29.  The output is (n, oh, ow, cout)."""
    if pad is None:
        pad = (kh // 2, kw // 2, kh // 2, kw // 2)
    oh = (h + pad[0] + pad[2] - dilation[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (w + pad[1] + pad[3] - dilation[1] * (kw - 1) - 1) // stride[1] + 1
    if oh <= 0 or ow <= 0 or oh % tile_h or ow % tile_w:
        raise ValueError("tile_h / tile_w must divide the output height / width")
    inp = Array(shape=(n, h, w, cin), dtype=dtype)
    filt = Array(shape=(kh, kw, cin, cout), dtype=dtype)
    out = Array(shape=(n, oh, ow, cout), dtype=float32)
    return convert(
        conv2d_kernel,
        args=(inp, filt, out, tile_h, tile_w, cin, cout, kh, kw, *pad, *stride, *dilation),
        grid=(n, oh // tile_h, ow // tile_w),
        double_buffering=True,
    )


# -- programs for the tile interpreter ----------------------------------------


@kernel
def layernorm_kernel(inp, gamma, beta, inv_n, eps, out, trow, col):
    """Row layernorm, the xt form of the reference's layernorm program
    (test/nova/to_x1.mlir:82-128: reduce, broadcast subtract, square, reduce,
    scale by 1/C plus epsilon, rsqrt, scale by gamma, add beta).  The DSL has
    no scalar operands, so 1/C and epsilon are (1, 1) tiles."""
    row = bid(0)
    x = load(inp, index=(row, 0), shape=(trow, col))
    g = load(gamma, index=(0, 0), shape=(1, col), shared=1)
    b = load(beta, index=(0, 0), shape=(1, col), shared=1)
    n = load(inv_n, index=(0, 0), shape=(1, 1), shared=1)
    e = load(eps, index=(0, 0), shape=(1, 1), shared=1)
    mean = tile_mul(tile_sum(x, axis=1), n)
    xc = tile_sub(x, mean)
    var = tile_mul(tile_sum(tile_mul(xc, xc), axis=1), n)
    r = rsqrt(tile_add(var, e))
    y = tile_add(tile_mul(tile_mul(xc, r), g), b)
    store(out, index=(row, 0), tile=y)


def layernorm(rows: int, cols: int, trow: int = 64):
    if rows % trow:
        raise ValueError("trow must divide rows")
    a = Array(shape=(rows, cols), dtype=float32)
    v = Array(shape=(1, cols), dtype=float32)
    s = Array(shape=(1, 1), dtype=float32)
    return convert(layernorm_kernel, args=(a, v, v, s, s, a, trow, cols), grid=(rows // trow, 1, 1),
                   double_buffering=True)


@kernel
def column_softmax_kernel(inp, out, row, tcol):
    """Softmax down the columns of a (row, tcol) tile: reductions over axis 0."""
    c = bid(0)
    x = load(inp, index=(0, c), shape=(row, tcol))
    m = tile_max(x, axis=0)
    ex = exp(tile_sub(x, m))
    y = tile_mul(ex, reciprocal(tile_sum(ex, axis=0)))
    store(out, index=(0, c), tile=y)


def column_softmax(rows: int, cols: int, tcol: int = 32):
    if cols % tcol:
        raise ValueError("tcol must divide cols")
    a = Array(shape=(rows, cols), dtype=float32)
    return convert(column_softmax_kernel, args=(a, a, rows, tcol), grid=(cols // tcol, 1, 1))


@kernel
def bias_add_kernel(inp, bias, out, trow, tcol):
    """x + bias with a (1, tcol) bias row broadcast over the tile's rows."""
    r = bid(0)
    c = bid(1)
    x = load(inp, index=(r, c), shape=(trow, tcol))
    b = load(bias, index=(0, c), shape=(1, tcol), shared=1)
    store(out, index=(r, c), tile=tile_add(x, b))


def bias_add(rows: int, cols: int, trow: int = 32, tcol: int = 64):
    a = Array(shape=(rows, cols), dtype=float32)
    v = Array(shape=(1, cols), dtype=float32)
    return convert(bias_add_kernel, args=(a, v, a, trow, tcol), grid=(rows // trow, cols // tcol, 1))


@kernel
def attention_kernel(q, k, v, o, tq, d, nk):
    """softmax(Q K^T) V for one query tile of one head: Q, V and the result
    are [heads, rows, d], K is [heads, nk, d].  The head's K and V tiles are
    shared by its query tiles (`shared = 1`); K^T comes from the DSL's rank-3
    transpose (xtile/dsl.py:426-438); P V multiplies the f32 probabilities by
    an f32 V, since matmul operands share a dtype (xtile/dsl.py:369-374)."""
    i = bid(0)
    h = bid(1)
    qt = reshape(load(q, index=(h, i, 0), shape=(1, tq, d)), shape=(tq, d))
    kt = load(k, index=(h, 0, 0), shape=(1, nk, d), shared=1)
    vt = reshape(load(v, index=(h, 0, 0), shape=(1, nk, d), shared=1), shape=(nk, d))
    ktt = reshape(transpose(kt), shape=(d, nk))
    s = matmul(qt, ktt)
    p = exp(tile_sub(s, tile_max(s, axis=1)))
    p = tile_mul(p, reciprocal(tile_sum(p, axis=1)))
    store(o, index=(h, i, 0), tile=reshape(matmul(p, vt), shape=(1, tq, d)))


def attention(heads: int, nq: int, nk: int, d: int, tq: int = 64, qk=float16):
    """Grid (nq / tq, heads, 1).  `qk` is the element type of Q and K (f16,
    bf16 or f32: their product is f32); V and the result are f32."""
    if nq % tq:
        raise ValueError("tq must divide nq")
    qa = Array(shape=(heads, nq, d), dtype=qk)
    ka = Array(shape=(heads, nk, d), dtype=qk)
    va = Array(shape=(heads, nk, d), dtype=float32)
    oa = Array(shape=(heads, nq, d), dtype=float32)
    return convert(attention_kernel, args=(qa, ka, va, oa, tq, d, nk), grid=(nq // tq, heads, 1))


CONFIGS = {
    "c1_add": lambda: add(1024, 1024, 32, 64),
    "c2_softmax": lambda: softmax(8192, 4096, 1),
    "c3_matmul_f16": lambda: matmul_f16(4096, 4096, 4096, 128, 128),
    "c4_conv2d_f16": lambda: conv2d(32, 56, 56, 64, 64, 3, 3, 4, 56),
    "c5_matmul_bf16": lambda: matmul_bf16(4096, 11008, 4096, 256, 128),
    "c6_matmul_i8": lambda: matmul_i8(4096, 4096, 4096, 64, 64),
}
