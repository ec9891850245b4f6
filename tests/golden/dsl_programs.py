"""Tile programs used to pin the DSL's emitted text.

`programs(xt)` builds each program against a DSL module `xt` that has the
reference API (kernel, bid, load, store, ...).  tests/golden/make_dsl_golden.py
runs them through the reference tracer (xtile/dsl.py) to write the expected
text; tests/test_dsl.py runs them through xtile_amd.dsl and compares.  Only
float32 / int8 programs appear here because those are the reference's dtypes
(xtile/dsl.py:14-15).  Sources of the programs: test/python/dsl_convert.py and
kernels/*.py of the reference, plus the benchmark configurations.
"""

from __future__ import annotations


def programs(xt):
    out = {}

    # test/python/dsl_convert.py:6-23
    @xt.kernel
    def rowwise_softmax(x, y):
        bid_x = xt.bid(0)
        t = xt.load(x, index=(bid_x, 0), shape=(64, 64))
        r = xt.max(t)
        t = t - r
        t = xt.exp(t)
        r = xt.sum(t)
        r = xt.reciprocal(r)
        t = t * r
        xt.store(y, index=(bid_x, 0), tile=t)

    a = xt.Array(shape=(128, 64), dtype=xt.float32)
    out["rowwise_softmax"] = (rowwise_softmax, (a, a), (2, 1, 1), True)

    # test/python/dsl_convert.py:46-83 (int8 matmul with scale/bias epilogue)
    @xt.kernel
    def matmul(lhs, rhs, res, scale, bias, tm, tn, tk):
        bid_x = xt.bid(0)
        bid_y = xt.bid(1)
        lhs_tile = xt.load(lhs, index=(bid_x, 0), shape=(tm, tk))
        rhs_tile = xt.load(rhs, index=(0, bid_y), shape=(tk, tn), shared=1)
        s_tile = xt.load(scale, index=(0, bid_y), shape=(1, tn), shared=1)
        b_tile = xt.load(bias, index=(0, bid_y), shape=(1, tn), shared=1)
        t = xt.matmul(lhs_tile, rhs_tile)
        t = t * s_tile + b_tile
        t = xt.astype(t, dtype=xt.int8)
        xt.store(res, index=(bid_x, bid_y), tile=t)

    out["matmul_int8_epilogue"] = (
        matmul,
        (
            xt.Array(shape=(1024, 256), dtype=xt.int8),
            xt.Array(shape=(256, 512), dtype=xt.int8),
            xt.Array(shape=(1024, 512), dtype=xt.int8),
            xt.Array(shape=(1, 512), dtype=xt.float32),
            xt.Array(shape=(1, 512), dtype=xt.float32),
            64,
            64,
            256,
        ),
        (16, 8, 1),
        True,
    )

    # test/python/dsl_convert.py:106-122
    @xt.kernel
    def divide_kernel(x, y, z):
        tile = xt.load(x, index=(0, 0), shape=(8, 8))
        denom = xt.load(y, index=(0, 0), shape=(8, 1))
        tile = tile / denom
        xt.store(z, index=(0, 0), tile=tile)

    out["divide_kernel"] = (
        divide_kernel,
        (
            xt.Array(shape=(8, 8), dtype=xt.float32),
            xt.Array(shape=(8, 1), dtype=xt.float32),
            xt.Array(shape=(8, 8), dtype=xt.float32),
        ),
        (1, 1, 1),
        False,
    )

    # test/python/dsl_convert.py:142-166
    @xt.kernel
    def load_conv2d_kernel(x, f, y):
        filt = xt.load(f, index=(0, 0, 0, 0), shape=(3, 3, 128, 64))
        tile = xt.load_conv2d(
            x,
            filt,
            index=(0, 0, 0, 0),
            shape=(1, 32, 64, 32),
            group=1,
            pad=(1, 1, 1, 1),
            stride=(1, 1),
            dilation=(1, 1),
        )
        xt.store(y, index=(0, 0, 0, 0), tile=tile)

    out["load_conv2d_kernel"] = (
        load_conv2d_kernel,
        (
            xt.Array(shape=(1, 34, 66, 128), dtype=xt.int8),
            xt.Array(shape=(3, 3, 128, 64), dtype=xt.int8),
            xt.Array(shape=(1, 32, 64, 32), dtype=xt.float32),
        ),
        (1, 1, 1),
        False,
    )

    # test/python/dsl_convert.py:186-214
    @xt.kernel
    def unary_and_shape(x, y, z, t_in, t_out):
        tile = xt.load(x, index=(0, 0), shape=(8, 8))
        tile = xt.cos(tile)
        tile = xt.sin(tile)
        tile = xt.rsqrt(tile)
        tile = xt.sigmoid(tile)
        tile = xt.tanh(tile)
        tile = xt.silu(tile)
        xt.store(y, index=(0, 0), tile=tile)
        reshaped = xt.reshape(tile, shape=(4, 16))
        xt.store(z, index=(0, 0), tile=reshaped)
        t3 = xt.load(t_in, index=(0, 0, 0), shape=(2, 3, 4))
        t3 = xt.transpose(t3)
        xt.store(t_out, index=(0, 0, 0), tile=t3)

    out["unary_and_shape"] = (
        unary_and_shape,
        (
            xt.Array(shape=(8, 8), dtype=xt.float32),
            xt.Array(shape=(8, 8), dtype=xt.float32),
            xt.Array(shape=(4, 16), dtype=xt.float32),
            xt.Array(shape=(2, 3, 4), dtype=xt.float32),
            xt.Array(shape=(2, 4, 3), dtype=xt.float32),
        ),
        (1, 1, 1),
        False,
    )

    # test/python/dsl_convert.py:229-247
    @xt.kernel
    def compute_ops(a, b, acc_src, acc_dst):
        a_tile = xt.load(a, index=(0, 0), shape=(16, 32))
        b_tile = xt.load(b, index=(0, 0), shape=(32, 8))
        acc_tile = xt.load(acc_src, index=(0, 0), shape=(16, 8))
        acc_tile = xt.mma(a_tile, b_tile, acc_tile)
        xt.store(acc_dst, index=(0, 0), tile=acc_tile)

    out["compute_ops"] = (
        compute_ops,
        (
            xt.Array(shape=(16, 32), dtype=xt.int8),
            xt.Array(shape=(32, 8), dtype=xt.int8),
            xt.Array(shape=(16, 8), dtype=xt.float32),
            xt.Array(shape=(16, 8), dtype=xt.float32),
        ),
        (1, 1, 1),
        False,
    )

    # test/python/dsl_convert.py:262-275
    @xt.kernel
    def column_reduce(x, y):
        tile = xt.load(x, index=(0, 0), shape=(8, 8))
        tile = xt.sum(tile, axis=0)
        xt.store(y, index=(0, 0), tile=tile)

    out["column_reduce"] = (
        column_reduce,
        (xt.Array(shape=(8, 8), dtype=xt.float32), xt.Array(shape=(1, 8), dtype=xt.float32)),
        (1, 1, 1),
        False,
    )

    # kernels/add.py:6-13 at --row 128 --col 128
    @xt.kernel
    def add_kernel(lhs, rhs, out_, trow, col):
        bid_x = xt.bid(0)
        a_ = xt.load(lhs, index=(bid_x, 0), shape=(trow, col))
        b_ = xt.load(rhs, index=(bid_x, 0), shape=(trow, col))
        c_ = a_ + b_
        xt.store(out_, index=(bid_x, 0), tile=c_)

    f128 = xt.Array(shape=(128, 128), dtype=xt.float32)
    out["add_kernel_rows"] = (add_kernel, (f128, f128, f128, 64, 128), (2, 1, 1), True)

    # benchmark C1: 32x64 tiles, grid (32, 16, 1)
    @xt.kernel
    def add_tiles(lhs, rhs, out_, tile_h, tile_w):
        b0 = xt.bid(0)
        b1 = xt.bid(1)
        a_ = xt.load(lhs, index=(b0, b1), shape=(tile_h, tile_w))
        b_ = xt.load(rhs, index=(b0, b1), shape=(tile_h, tile_w))
        xt.store(out_, index=(b0, b1), tile=a_ + b_)

    f1k = xt.Array(shape=(1024, 1024), dtype=xt.float32)
    out["c1_add"] = (add_tiles, (f1k, f1k, f1k, 32, 64), (32, 16, 1), True)

    # kernels/softmax.py:10-19 at the C2 shape with one row per Block
    @xt.kernel
    def softmax_kernel(inp, out_, trow, col):
        bid_x = xt.bid(0)
        x = xt.load(inp, index=(bid_x, 0), shape=(trow, col))
        x = x - xt.max(x, axis=-1)
        x = xt.exp(x)
        r = xt.sum(x, axis=-1)
        x = x / r
        xt.store(out_, index=(bid_x, 0), tile=x)

    s = xt.Array(shape=(8192, 4096), dtype=xt.float32)
    out["c2_softmax"] = (softmax_kernel, (s, s, 1, 4096), (8192, 1, 1), True)

    # kernels/conv2d.py:10-37 at its defaults (int8)
    @xt.kernel
    def conv2d_kernel(inp, filt, out_, tile_h, tile_w, cin, cout, kh, kw):
        bid_n = xt.bid(0)
        bid_h = xt.bid(1)
        bid_w = xt.bid(2)
        zero = 0
        filt_tile = xt.load(filt, index=(zero, zero, zero, zero), shape=(kh, kw, cin, cout), shared=2)
        out_tile = xt.load_conv2d(
            inp,
            filt_tile,
            index=(bid_n, bid_h, bid_w, zero),
            shape=(1, tile_h, tile_w, cout),
            group=1,
            pad=(kh // 2, kw // 2, kh // 2, kw // 2),
            stride=(1, 1),
            dilation=(1, 1),
        )
        xt.store(out_, index=(bid_n, bid_h, bid_w, zero), tile=out_tile)

    out["conv2d_kernel_int8"] = (
        conv2d_kernel,
        (
            xt.Array(shape=(1, 32, 64, 128), dtype=xt.int8),
            xt.Array(shape=(3, 3, 128, 64), dtype=xt.int8),
            xt.Array(shape=(1, 32, 64, 64), dtype=xt.float32),
            32,
            64,
            128,
            64,
            3,
            3,
        ),
        (1, 1, 1),
        True,
    )

    # a program that exercises constant naming beyond %zero (%c1, %c2, %c3)
    @xt.kernel
    def const_coords(x, y):
        t = xt.load(x, index=(1, 2), shape=(4, 8))
        u = xt.load(x, index=(3, 1), shape=(4, 8))
        xt.store(y, index=(2, 0), tile=t + u)

    out["const_coords"] = (
        const_coords,
        (xt.Array(shape=(16, 24), dtype=xt.float32), xt.Array(shape=(16, 24), dtype=xt.float32)),
        (1, 1, 1),
        False,
    )
    return out
