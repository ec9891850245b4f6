"""Seeded random xt tile programs for the tile interpreter's parity tests.

Each program loads one or two row tiles per Block (f32, f16, bf16 or i8
memrefs), combines them with broadcast add / sub / mul, applies bounded unary
ops, reduces along an axis, optionally transposes (through a rank-3 reshape)
or multiplies by a loaded matrix, and stores an f32 result.  Values stay
bounded (inputs in [-1, 1], exp of values <= 4) so that no program overflows,
and the shapes keep every live tile small.

`program(seed)` returns (xt text, host input arrays, dtypes, output index,
output shape).
"""

from __future__ import annotations

import numpy as np

from oracle import f32_to_bf16_bits

_ELEMS = ["f32", "f16", "bf16", "i8"]
_UNARY = ["xt.exp", "xt.sin", "xt.cos", "xt.tanh", "xt.sigmoid", "xt.silu"]


def _t(shape, e="f32"):
    return "tensor<" + "x".join(map(str, shape)) + "x" + e + ">"


def _m(shape, e="f32"):
    return "memref<" + "x".join(map(str, shape)) + "x" + e + ">"


def _host(rng, shape, e):
    if e == "i8":  # small integers keep exp of them (+ a uniform operand) at most e^4
        return rng.integers(-3, 4, shape, dtype=np.int8)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    if e == "f16":
        return x.astype(np.float16)
    if e == "bf16":
        return f32_to_bf16_bits(x)
    return x


def program(seed: int):
    rng = np.random.default_rng(seed)
    grid = int(rng.integers(1, 5))
    R = int(rng.choice([2, 4, 8, 16]))
    C = int(rng.choice([4, 8, 16, 32, 64]))
    ea = str(rng.choice(_ELEMS))
    rows = grid * R
    lines, args, host, dtypes = [], [], [], []
    n = [0]

    def fresh():
        n[0] += 1
        return f"%v{n[0]}"

    def add_arg(shape, e):
        name = f"%a{len(args)}"
        args.append(f"{name}: {_m(shape, e)}")
        host.append(_host(rng, shape, e))
        dtypes.append(e)
        return name

    # x: the Block's R x C row tile of A
    A = add_arg((rows, C), ea)
    x = fresh()
    lines.append(f"  {x} = xt.load({A}, %bid#0, %z) : ({_m((rows, C), ea)}, i32, i32) -> {_t((R, C), ea)}")
    cur, cur_e, shape = x, ea, (R, C)
    if ea == "i8":  # bring it to f32 (itof), the dialect's cast
        y = fresh()
        lines.append(f"  {y} = xt.itof({cur}) : {_t(shape, 'i8')} -> {_t(shape)}")
        cur, cur_e = y, "f32"
    # a broadcast operand: (1, C), (R, 1) or (R, C), f32, shared along the grid when it is a row
    kind = int(rng.integers(0, 3))
    bshape = [(1, C), (R, 1), (R, C)][kind]
    bmem = (1, C) if kind == 0 else (rows, bshape[1])
    Bn = add_arg(bmem, "f32")
    b = fresh()
    coords = "%z, %z" if kind == 0 else "%bid#0, %z"
    shared = " {shared = 1 : i64}" if kind == 0 else ""
    lines.append(f"  {b} = xt.load({Bn}, {coords}){shared} : ({_m(bmem)}, i32, i32) -> {_t(bshape)}")
    if cur_e != "f32":  # f16 / bf16 tiles combine with f16 / bf16 operands only; use the load as is
        y = fresh()
        op = str(rng.choice(["xt.add", "xt.sub", "xt.mul"]))
        lines.append(f"  {y} = {op}({cur}, {cur}) : {_t(shape, cur_e)}, {_t(shape, cur_e)} -> {_t(shape, cur_e)}")
        cur = y
        # store this narrow tile too (rounded like the oracle), then continue from f32 b
        On = add_arg((rows, C), cur_e)
        lines.append(f"  xt.store({cur}, {On}, %bid#0, %z) : ({_t(shape, cur_e)}, {_m((rows, C), cur_e)}, i32, i32) -> ()")
        y = fresh()
        lines.append(f"  {y} = xt.mul({b}, {b}) : {_t(bshape)}, {_t(bshape)} -> {_t(bshape)}")
        cur, shape = y, bshape
    else:
        y = fresh()
        op = str(rng.choice(["xt.add", "xt.sub", "xt.mul"]))
        lines.append(f"  {y} = {op}({cur}, {b}) : {_t(shape)}, {_t(bshape)} -> {_t(shape)}")
        cur = y
    # one or two bounded unary ops
    for _ in range(int(rng.integers(1, 3))):
        y = fresh()
        u = str(rng.choice(_UNARY))
        lines.append(f"  {y} = {u}({cur}) : {_t(shape)} -> {_t(shape)}")
        cur = y
    # a keep-dim reduction broadcast back (rank 2 only)
    if shape[0] > 1 and shape[1] > 1 and rng.random() < 0.7:
        axis = int(rng.integers(0, 2))
        red = str(rng.choice(["xt.reduce_sum", "xt.reduce_max"]))
        rs = (1, shape[1]) if axis == 0 else (shape[0], 1)
        r = fresh()
        lines.append(f"  {r} = {red}({cur}) {{axis = {axis} : i64}} : {_t(shape)} -> {_t(rs)}")
        y = fresh()
        lines.append(f"  {y} = xt.sub({cur}, {r}) : {_t(shape)}, {_t(rs)} -> {_t(shape)}")
        cur = y
    # optionally a matmul by a loaded (C', N) matrix, or a transpose of the last two dims
    tail = rng.random()
    if tail < 0.35:
        N = int(rng.choice([4, 8, 16]))
        Wn = add_arg((shape[1], N), "f32")
        w = fresh()
        lines.append(f"  {w} = xt.load({Wn}, %z, %z) {{shared = 1 : i64}} : ({_m((shape[1], N))}, i32, i32) -> {_t((shape[1], N))}")
        y = fresh()
        lines.append(f"  {y} = xt.matmul({cur}, {w}) : {_t(shape)}, {_t((shape[1], N))} -> {_t((shape[0], N))}")
        cur, shape = y, (shape[0], N)
    elif tail < 0.6:
        r3 = fresh()
        lines.append(f"  {r3} = xt.reshape({cur}) : {_t(shape)} -> {_t((1,) + shape)}")
        t3 = fresh()
        lines.append(f"  {t3} = xt.transpose({r3}) : {_t((1,) + shape)} -> {_t((1, shape[1], shape[0]))}")
        y = fresh()
        lines.append(f"  {y} = xt.reshape({t3}) : {_t((1, shape[1], shape[0]))} -> {_t((shape[1], shape[0]))}")
        cur, shape = y, (shape[1], shape[0])
    out_shape = (grid * shape[0], shape[1])
    On = add_arg(out_shape, "f32")
    host[-1] = np.zeros(out_shape, np.float32)
    lines.append(f"  xt.store({cur}, {On}, %bid#0, %z) : ({_t(shape)}, {_m(out_shape)}, i32, i32) -> ()")
    head = (f"func.func @rnd{seed}({', '.join(args)}) attributes {{xt.grid = array<i32: {grid}, 1, 1>}} {{\n"
            "  %bid:3 = xt.get_tile_block_id : i32, i32, i32\n  %z = arith.constant 0 : i32\n")
    text = head + "\n".join(lines) + "\n  func.return\n}"
    # narrow intermediate outputs start at zero too
    for k, d in enumerate(dtypes):
        if k > 0 and k != len(dtypes) - 1 and host[k].shape == (rows, C) and d == ea and d != "f32":
            host[k] = np.zeros_like(host[k])
    return text, host, dtypes, len(dtypes) - 1


# (R, C) tiles of the fused kernel's layouts: rows across up to 8 waves, several
# rows per thread, tall tiles whose column reductions span many threads
_FUSED_TILES = [(1, 4096), (2, 2048), (4, 1024), (8, 512), (16, 256), (64, 64), (128, 32), (256, 8), (3, 20), (6, 12)]


def fused_program(seed: int):
    """A random program over one [R, C] tile and its broadcasts, the form the
    fused kernel takes: a loaded tile (any element type), a shared [1, C]
    weight and [1, 1] scalar, a per-Block [R, 1] operand, bounded unary ops,
    keep-dim reductions broadcast back (max subtracted, sum multiplied), and stores of the f32 result and of a
    reduction.  Grids up to 6000 Blocks, so that workgroups walk several Blocks
    with the shared tiles in registers.  Returns (text, host arrays, dtypes,
    indices of the f32 outputs)."""
    rng = np.random.default_rng(10_000 + seed)
    R, C = _FUSED_TILES[int(rng.integers(0, len(_FUSED_TILES)))]
    big = rng.random() < 0.3 and R * C <= 4096
    grid = int(rng.integers(4097, 6001)) if big else int(rng.integers(1, 9))
    rows = grid * R
    ea = str(rng.choice(_ELEMS))
    lines, args, host, dtypes, outs = [], [], [], [], []
    n = [0]

    def fresh():
        n[0] += 1
        return f"%v{n[0]}"

    def add_arg(shape, e, out=False):
        args.append(f"%a{len(args)}: {_m(shape, e)}")
        host.append(np.zeros(shape, np.float32) if out else _host(rng, shape, e))
        dtypes.append(e)
        if out:
            outs.append(len(args) - 1)
        return f"%a{len(args) - 1}"

    A = add_arg((rows, C), ea)
    x = fresh()
    lines.append(f"  {x} = xt.load({A}, %bid#0, %z) : ({_m((rows, C), ea)}, i32, i32) -> {_t((R, C), ea)}")
    if ea == "i8":
        y = fresh()
        lines.append(f"  {y} = xt.itof({x}) : {_t((R, C), 'i8')} -> {_t((R, C))}")
        x = y
    elif ea != "f32":  # f16 / bf16 values combine with their own type; square, then restart from an f32 load
        y = fresh()
        lines.append(f"  {y} = xt.mul({x}, {x}) : {_t((R, C), ea)}, {_t((R, C), ea)} -> {_t((R, C), ea)}")
        On = add_arg((rows, C), ea)
        host[-1] = np.zeros_like(host[-1])
        lines.append(f"  xt.store({y}, {On}, %bid#0, %z) : ({_t((R, C), ea)}, {_m((rows, C), ea)}, i32, i32) -> ()")
        F = add_arg((rows, C), "f32")
        x = fresh()
        lines.append(f"  {x} = xt.load({F}, %bid#0, %z) : ({_m((rows, C))}, i32, i32) -> {_t((R, C))}")
    W = add_arg((1, C), "f32")
    w = fresh()
    lines.append(f"  {w} = xt.load({W}, %z, %z) {{shared = 1 : i64}} : ({_m((1, C))}, i32, i32) -> {_t((1, C))}")
    S = add_arg((1, 1), "f32")
    sc = fresh()
    lines.append(f"  {sc} = xt.load({S}, %z, %z) {{shared = 1 : i64}} : ({_m((1, 1))}, i32, i32) -> {_t((1, 1))}")
    P = add_arg((rows, 1), "f32")
    pr = fresh()
    lines.append(f"  {pr} = xt.load({P}, %bid#0, %z) : ({_m((rows, 1))}, i32, i32) -> {_t((R, 1))}")
    cur = x
    ops = ["xt.add", "xt.sub", "xt.mul"]
    for operand, shape in [(w, (1, C)), (sc, (1, 1)), (pr, (R, 1))]:
        y = fresh()
        lines.append(f"  {y} = {rng.choice(ops)}({cur}, {operand}) : {_t((R, C))}, {_t(shape)} -> {_t((R, C))}")
        cur = y
    y = fresh()
    lines.append(f"  {y} = {rng.choice(_UNARY)}({cur}) : {_t((R, C))} -> {_t((R, C))}")
    cur = y
    red_out = None
    for _ in range(int(rng.integers(1, 3))):
        axis = int(rng.integers(0, 2))
        rs = (1, C) if axis == 0 else (R, 1)
        r = fresh()
        red = str(rng.choice(["xt.reduce_sum", "xt.reduce_max"]))
        lines.append(f"  {r} = {red}({cur}) {{axis = {axis} : i64}} : {_t((R, C))} -> {_t(rs)}")
        # a max is subtracted (exact); a sum scales (a difference from a sum of C values would cancel)
        y = fresh()
        op = "xt.sub" if red == "xt.reduce_max" else "xt.mul"
        lines.append(f"  {y} = {op}({cur}, {r}) : {_t((R, C))}, {_t(rs)} -> {_t((R, C))}")
        cur = y
        red_out = (r, rs)
    r, rs = red_out
    mem = (grid, C) if rs[0] == 1 else (rows, 1)
    Rn = add_arg(mem, "f32", out=True)
    lines.append(f"  xt.store({r}, {Rn}, %bid#0, %z) : ({_t(rs)}, {_m(mem)}, i32, i32) -> ()")
    On = add_arg((rows, C), "f32", out=True)
    lines.append(f"  xt.store({cur}, {On}, %bid#0, %z) : ({_t((R, C))}, {_m((rows, C))}, i32, i32) -> ()")
    head = (f"func.func @fz{seed}({', '.join(args)}) attributes {{xt.grid = array<i32: {grid}, 1, 1>}} {{\n"
            "  %bid:3 = xt.get_tile_block_id : i32, i32, i32\n  %z = arith.constant 0 : i32\n")
    return head + "\n".join(lines) + "\n  func.return\n}", host, dtypes, outs


def conv_case(seed: int):
    """Random `load_conv2d` parameters the planner takes (any kernel): element
    type, batch, image, channels, filter, asymmetric pads, strides, dilations,
    and output tiles dividing the output.  Returns (module, host inputs,
    dtypes, description); the module is built by xtile_amd.kernels.conv2d."""
    import xtile_amd as xt
    from xtile_amd import kernels as K

    rng = np.random.default_rng(20_000 + seed)
    dts = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}
    for _ in range(200):
        dt = str(rng.choice(list(dts)))
        n = int(rng.integers(1, 3))
        kh, kw = int(rng.choice([1, 3, 5])), int(rng.choice([1, 3, 5]))
        sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        dh, dw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        pad = tuple(int(rng.integers(0, k // 2 + 1)) for k in (kh, kw, kh, kw))
        h, w = int(rng.integers(6, 21)), int(rng.integers(6, 21))
        cin = int(rng.choice([3, 8, 16, 32, 48, 64, 96, 128]))
        cout = int(rng.choice([8, 16, 24, 32, 48, 64, 128]))
        oh = (h + pad[0] + pad[2] - dh * (kh - 1) - 1) // sh + 1
        ow = (w + pad[1] + pad[3] - dw * (kw - 1) - 1) // sw + 1
        if oh < 1 or ow < 1:
            continue
        th = int(rng.choice([d for d in range(1, oh + 1) if oh % d == 0]))
        tw = int(rng.choice([d for d in range(1, ow + 1) if ow % d == 0]))
        try:
            mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=dts[dt], pad=pad, stride=(sh, sw),
                           dilation=(dh, dw))
            xt.plan(mod)
        except (ValueError, NotImplementedError):
            continue
        if dt == "i8":
            x = rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8)
            f = rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8)
        else:
            x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
            f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
            x, f = (f32_to_bf16_bits(x), f32_to_bf16_bits(f)) if dt == "bf16" else (x.astype(np.float16),
                                                                                     f.astype(np.float16))
        o = np.zeros((n, oh, ow, cout), np.float32)
        desc = (f"{dt} {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{sh},{sw} d{dh},{dw} pad{pad} "
                f"tile {th}x{tw}")
        return mod, [x, f, o], [dt, dt, "f32"], desc
    raise RuntimeError("no plannable conv drawn")


def wide_conv_case(seed: int):
    """Random `load_conv2d` programs in the implicit-GEMM kernel's range: Blocks
    tiling the whole output, Cin and Cout multiples of 8 (16 for i8) up to 320
    and 256, 1x1 to 5x5 filters, strides, dilations and asymmetric pads.
    Returns (module, host inputs, dtypes, description)."""
    import xtile_amd as xt
    from xtile_amd import kernels as K

    rng = np.random.default_rng(25_000 + seed)
    dts = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}
    for _ in range(200):
        dt = str(rng.choice(list(dts)))
        q = 16 if dt == "i8" else 8
        n = int(rng.integers(1, 3))
        kh, kw = int(rng.choice([1, 3, 5])), int(rng.choice([1, 3, 5]))
        sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        dh, dw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        pad = tuple(int(rng.integers(0, k // 2 + 1)) for k in (kh, kw, kh, kw))
        h, w = int(rng.integers(5, 17)), int(rng.integers(5, 17))
        cin = q * int(rng.integers(1, 320 // q + 1))
        cout = q * int(rng.integers(1, 256 // q + 1))
        oh = (h + pad[0] + pad[2] - dh * (kh - 1) - 1) // sh + 1
        ow = (w + pad[1] + pad[3] - dw * (kw - 1) - 1) // sw + 1
        if oh < 1 or ow < 1:
            continue
        th = int(rng.choice([d for d in range(1, oh + 1) if oh % d == 0]))
        tw = int(rng.choice([d for d in range(1, ow + 1) if ow % d == 0]))
        try:
            mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=dts[dt], pad=pad, stride=(sh, sw),
                           dilation=(dh, dw))
            xt.plan(mod)
        except (ValueError, NotImplementedError):
            continue
        if dt == "i8":
            x = rng.integers(-128, 128, (n, h, w, cin), dtype=np.int8)
            f = rng.integers(-128, 128, (kh, kw, cin, cout), dtype=np.int8)
        else:
            x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
            f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
            x, f = (f32_to_bf16_bits(x), f32_to_bf16_bits(f)) if dt == "bf16" else (x.astype(np.float16),
                                                                                     f.astype(np.float16))
        o = np.zeros((n, oh, ow, cout), np.float32)
        desc = (f"{dt} {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s{sh},{sw} d{dh},{dw} pad{pad} "
                f"tile {th}x{tw}")
        return mod, [x, f, o], [dt, dt, "f32"], desc
    raise RuntimeError("no plannable conv drawn")


def wide_gemm_case(seed: int):
    """Random matmul programs for the DMA kernel's tile choice: M and N
    multiples of 128 up to 2048 (odd multiples included, so 256 x 128, 128 x
    256 and 128 x 128 tiles and the K split all occur), K multiples of 128 up
    to 2048, 64 x 64 Block tiles, f32 results of f16 / bf16 (some with scale
    and bias) and the i8 epilogue with an i8 result.  Returns (module, host
    inputs, dtypes, output index, description)."""
    import xtile_amd as xt
    from xtile_amd import Array, bid, cdiv, convert, float32, int8, kernel, load, matmul, store, astype

    rng = np.random.default_rng(35_000 + seed)
    dt = str(rng.choice(["f16", "bf16", "i8"]))
    while True:
        m, n, k = 128 * int(rng.integers(1, 17)), 128 * int(rng.integers(1, 17)), 128 * int(rng.integers(1, 17))
        if m * n * k <= 2**31:
            break
    epi = dt == "i8" or bool(rng.random() < 0.4)
    ftoi = dt == "i8"

    @kernel
    def prog(lhs, rhs, res, sc, bi, tm, tn, tk):
        x = bid(0)
        y = bid(1)
        t = matmul(load(lhs, index=(x, 0), shape=(tm, tk)), load(rhs, index=(0, y), shape=(tk, tn), shared=1))
        if epi:
            t = t * load(sc, index=(0, y), shape=(1, tn), shared=1)
            t = t + load(bi, index=(0, y), shape=(1, tn), shared=1)
        if ftoi:
            t = astype(t, dtype=int8)
        store(res, index=(x, y), tile=t)

    dt_in = {"i8": xt.int8, "f16": xt.float16, "bf16": xt.bfloat16}[dt]
    args = (Array(shape=(m, k), dtype=dt_in), Array(shape=(k, n), dtype=dt_in),
            Array(shape=(m, n), dtype=int8 if ftoi else float32), Array(shape=(1, n), dtype=float32),
            Array(shape=(1, n), dtype=float32), 64, 64, k)
    mod = convert(prog, args=args, grid=(cdiv(m, 64), cdiv(n, 64), 1))
    if dt == "i8":
        a = rng.integers(-128, 128, (m, k), dtype=np.int8)
        b = rng.integers(-128, 128, (k, n), dtype=np.int8)
        s = (rng.uniform(0.5, 2.0, (1, n)) / (np.sqrt(k) * 64)).astype(np.float32)
        bias = rng.uniform(-20, 20, (1, n)).astype(np.float32)
    else:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        a, b = (a.astype(np.float16), b.astype(np.float16)) if dt == "f16" else (f32_to_bf16_bits(a),
                                                                               f32_to_bf16_bits(b))
        s = rng.uniform(0.5, 2.0, (1, n)).astype(np.float32)
        bias = rng.uniform(-2, 2, (1, n)).astype(np.float32)
    c = np.zeros((m, n), np.int8 if ftoi else np.float32)
    desc = f"{dt} {m}x{n}x{k} epilogue={epi} ftoi={ftoi}"
    return mod, [a, b, c, s, bias], [dt, dt, "i8" if ftoi else "f32", "f32", "f32"], 2, desc


def gemm_case(seed: int):
    """A random matmul program of xtile_amd.kernels: f16 / bf16 (f32 result)
    or the i8 epilogue form (i8 result of A @ B * scale + bias), M, N, K
    multiples of 64 up to 1024 (K of 128 for i8), Block tiles of 64, 128 or 256 dividing them.
    Returns (module, host inputs, dtypes, output index, description)."""
    from xtile_amd import kernels as K

    rng = np.random.default_rng(30_000 + seed)
    dt = str(rng.choice(["f16", "bf16", "i8"]))
    m, n, k = (64 * int(rng.integers(1, 17)) for _ in range(3))
    if dt == "i8":  # the i8 MFMA steps K by 128 (32x32x32, two steps in flight)
        k = 128 * max(1, k // 128)
    tm = int(rng.choice([t for t in (64, 128, 256) if m % t == 0]))
    tn = int(rng.choice([t for t in (64, 128, 256) if n % t == 0]))
    desc = f"{dt} {m}x{n}x{k} tile {tm}x{tn}"
    if dt == "i8":
        a = rng.integers(-128, 128, (m, k), dtype=np.int8)
        b = rng.integers(-128, 128, (k, n), dtype=np.int8)
        s = (rng.uniform(0.5, 2.0, (1, n)) / (np.sqrt(k) * 64)).astype(np.float32)
        bias = rng.uniform(-20, 20, (1, n)).astype(np.float32)
        return K.matmul_i8(m, n, k, tm, tn), [a, b, np.zeros((m, n), np.int8), s, bias], \
            ["i8", "i8", "i8", "f32", "f32"], 2, desc
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    if dt == "f16":
        mod, a, b = K.matmul_f16(m, n, k, tm, tn), a.astype(np.float16), b.astype(np.float16)
    else:
        mod, a, b = K.matmul_bf16(m, n, k, tm, tn), f32_to_bf16_bits(a), f32_to_bf16_bits(b)
    return mod, [a, b, np.zeros((m, n), np.float32)], [dt, dt, "f32"], 2, desc


def stream_case(seed: int):
    """A random program of the two streaming families: f32 add over 2-D tiles
    (any tile dividing the array, odd sizes included) or row softmax with
    full-width row tiles of 1-16 rows and 1-8192 columns.  Returns (module,
    host inputs, dtypes, output index, description)."""
    from xtile_amd import kernels as K

    rng = np.random.default_rng(40_000 + seed)

    def divisor(v):
        return int(rng.choice([d for d in range(1, min(v, 256) + 1) if v % d == 0]))

    if rng.random() < 0.5:
        rows, cols = int(rng.integers(1, 1025)), int(rng.integers(1, 1025))
        th, tw = divisor(rows), divisor(cols)
        a = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
        b = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
        return K.add(rows, cols, th, tw), [a, b, np.zeros_like(a)], ["f32"] * 3, 2, \
            f"add {rows}x{cols} tile {th}x{tw}"
    import xtile_amd as xt

    for _ in range(100):  # long rows that are not float4-aligned go elsewhere or are refused: draw again
        cols = int(rng.choice([int(rng.integers(1, 8193)), 2048 * int(rng.integers(1, 5)),
                               64 * int(rng.integers(1, 65))]))
        trow = int(rng.choice([1, 2, 4, 8, 16]))
        rows = trow * int(rng.integers(1, 65))
        mod = K.softmax(rows, cols, trow)
        if xt.plan(mod)["kernel"].startswith("row_softmax") if _plans(mod) else False:
            break
    x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
    return mod, [x, np.zeros_like(x)], ["f32"] * 2, 1, f"softmax {rows}x{cols} tile {trow}x{cols}"


def _plans(mod) -> bool:
    import xtile_amd as xt

    try:
        xt.plan(mod)
        return True
    except NotImplementedError:
        return False


def image_conv_case(seed: int):
    """Random `load_conv2d` programs in the resident-image kernel's range
    (conv_image.hip): f16 / bf16, Blocks tiling the whole output, Cin a
    multiple of 64 up to 256, Cout a multiple of 32 up to 256, a 3-wide filter
    of height 1, 3 or 5, strides and dilations of 1 or 2, asymmetric pads, at
    most 256 outputs an image, and the image's channels (144-byte pixels, 7 a
    DMA instruction) plus four 12 KB filter stages within 160 KB of LDS.
    Returns (module, host inputs, dtypes, description)."""
    import xtile_amd as xt
    from xtile_amd import kernels as K

    rng = np.random.default_rng(27_000 + seed)
    for _ in range(500):
        dt = str(rng.choice(["f16", "bf16"]))
        n = int(rng.integers(1, 3))
        kh, kw = int(rng.choice([1, 3, 5])), 3
        sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        dh, dw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        pad = tuple(int(rng.integers(0, k // 2 + 1)) for k in (kh, kw, kh, kw))
        h, w = int(rng.integers(5, 17)), int(rng.integers(5, 17))
        cin, cout = 64 * int(rng.integers(1, 5)), 32 * int(rng.integers(1, 9))
        oh = (h + pad[0] + pad[2] - dh * (kh - 1) - 1) // sh + 1
        ow = (w + pad[1] + pad[3] - dw * (kw - 1) - 1) // sw + 1
        if oh < 1 or ow < 1 or oh * ow > 256:
            continue
        mt = (oh * ow + 31) // 32
        region = (h * w + 6) // 7 * 1008 + 16
        if max(cin // 64 * region + 256 + 4 * 12288, 16 * mt * 1024) > 160 * 1024:
            continue
        th = int(rng.choice([d for d in range(1, oh + 1) if oh % d == 0]))
        tw = int(rng.choice([d for d in range(1, ow + 1) if ow % d == 0]))
        try:
            mod = K.conv2d(n, h, w, cin, cout, kh, kw, th, tw, dtype=xt.bfloat16 if dt == "bf16" else xt.float16,
                           pad=pad, stride=(sh, sw), dilation=(dh, dw))
            xt.plan(mod)
        except (ValueError, NotImplementedError):
            continue
        x = rng.normal(0, 0.1, (n, h, w, cin)).astype(np.float32)
        f = rng.normal(0, 0.1, (kh, kw, cin, cout)).astype(np.float32)
        x, f = (f32_to_bf16_bits(x), f32_to_bf16_bits(f)) if dt == "bf16" else (x.astype(np.float16),
                                                                                 f.astype(np.float16))
        o = np.full((n, oh, ow, cout), 7.0, np.float32)
        desc = (f"{dt} {n}x{h}x{w}x{cin}->{cout} k{kh}x{kw} s({sh},{sw}) d({dh},{dw}) pad{pad} "
                f"tile {th}x{tw}")
        return mod, [x, f, o], [dt, dt, "f32"], desc
    raise RuntimeError(f"no resident-image conv case for seed {seed}")
