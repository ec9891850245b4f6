"""TEST INFRASTRUCTURE: literal restatement of the serialized program.

Follows lib/xt/XTSerialize.cpp:63-104 step by step rather than through the
closed form the C executor uses: blocks run in z -> y -> x order; a load with
`shared = k > 0` is evaluated only for the first block whose key
(load, y if k == 1 else 0, z) has not been seen, and every later block of that
key reuses the cached tile.  Small grids only (pure Python over blocks, numpy
per op).  Tests compare it against the C executor to pin the sharing rule.
"""

from __future__ import annotations

import numpy as np

from . import bf16_bits_to_f32, f32_to_bf16_bits
from .xt_reader import RFunc, read_function


def _read(buf: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(buf)
    return buf.astype(np.float32)


def _write(dtype: str, values: np.ndarray) -> np.ndarray:
    if dtype == "bf16":
        return f32_to_bf16_bits(values.astype(np.float32))
    if dtype == "i8":
        return np.clip(np.rint(values), -128, 127).astype(np.int8)
    if dtype == "f16":
        return values.astype(np.float16)
    return values.astype(np.float32)


def _slices(coords, shape):
    return tuple(slice(c * s, c * s + s) for c, s in zip(coords, shape))


def run(text: str, buffers, func: str | None = None) -> None:
    fn: RFunc = read_function(text, func)
    args = {name: k for k, (name, _) in enumerate(fn.args)}
    dtypes = [t.dtype for _, t in fn.args]
    gx, gy, gz = fn.grid
    shared_cache: dict[tuple[int, int, int], np.ndarray] = {}
    for z in range(gz):
        for y in range(gy):
            for x in range(gx):
                env: dict[str, object] = {}
                for k, op in enumerate(fn.ops):
                    name = op.name
                    if name == "xt.get_tile_block_id":
                        for r, v in zip(op.results, (x, y, z)):
                            env[r] = v
                    elif name == "arith.constant":
                        env[op.results[0]] = int(op.attrs["value"])
                    elif name == "xt.load":
                        shared = int(op.attrs.get("shared", 0))
                        key = (k, y if shared == 1 else 0, z)
                        if shared > 0 and key in shared_cache:
                            env[op.results[0]] = shared_cache[key]
                            continue
                        a = args[op.operands[0]]
                        coords = [env[c] for c in op.operands[1:]]
                        tile = _read(buffers[a][_slices(coords, op.result_type.shape)], dtypes[a])
                        if tile.shape != op.result_type.shape:
                            raise IndexError("load out of bounds")
                        env[op.results[0]] = tile
                        if shared > 0:
                            shared_cache[key] = tile
                    elif name == "xt.store":
                        a = args[op.operands[1]]
                        coords = [env[c] for c in op.operands[2:]]
                        val = env[op.operands[0]]
                        buffers[a][_slices(coords, val.shape)] = _write(dtypes[a], val)
                    elif name == "xt.load_conv2d":
                        a = args[op.operands[0]]
                        src = _read(buffers[a], dtypes[a]).astype(np.float64)
                        filt = np.asarray(env[op.operands[1]], dtype=np.float64)
                        cb, ch, cw, cc = (env[c] for c in op.operands[2:])
                        tb, th, tw, tc = op.result_type.shape
                        kh_n, kw_n, cin, _ = filt.shape
                        pt, pl = op.attrs["pad"][0], op.attrs["pad"][1]
                        sh, sw = op.attrs["stride"]
                        dh, dw = op.attrs["dilation"]
                        out = np.zeros((tb, th, tw, tc))
                        for b in range(tb):
                            for i in range(th):
                                for j in range(tw):
                                    for kh in range(kh_n):
                                        ih = (ch * th + i) * sh - pt + kh * dh
                                        if not 0 <= ih < src.shape[1]:
                                            continue
                                        for kw in range(kw_n):
                                            iw = (cw * tw + j) * sw - pl + kw * dw
                                            if not 0 <= iw < src.shape[2]:
                                                continue
                                            vec = src[cb * tb + b, ih, iw, cc * cin : cc * cin + cin]
                                            out[b, i, j] += vec @ filt[kh, kw, :, :tc]
                        env[op.results[0]] = out.astype(np.float32)
                    else:
                        vals = [env[o] for o in op.operands]
                        env[op.results[0]] = _compute(name, vals, op)
    return None


def _compute(name: str, vals, op) -> np.ndarray:
    f32 = np.float32
    if name in ("xt.add", "xt.sub", "xt.mul"):
        a, b = (np.asarray(v, dtype=f32) for v in vals)
        return {"xt.add": np.add, "xt.sub": np.subtract, "xt.mul": np.multiply}[name](a, b).astype(f32)
    a = np.asarray(vals[0], dtype=f32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if name == "xt.exp":
            return np.exp(a).astype(f32)
        if name == "xt.cos":
            return np.cos(a).astype(f32)
        if name == "xt.sin":
            return np.sin(a).astype(f32)
        if name == "xt.reciprocal":
            return (f32(1.0) / a).astype(f32)
        if name == "xt.rsqrt":
            return (f32(1.0) / np.sqrt(a)).astype(f32)
        if name == "xt.sigmoid":
            return (f32(1.0) / (f32(1.0) + np.exp(-a))).astype(f32)
        if name == "xt.tanh":
            return np.tanh(a).astype(f32)
        if name == "xt.silu":
            return (a * (f32(1.0) / (f32(1.0) + np.exp(-a)))).astype(f32)
    if name == "xt.itof":
        return a
    if name == "xt.ftoi":
        return np.clip(np.rint(a), -128, 127).astype(f32)
    if name in ("xt.reduce_sum", "xt.reduce_max"):
        axis = int(op.attrs["axis"]) % a.ndim
        if name == "xt.reduce_max":
            return np.max(a, axis=axis, keepdims=True)
        # sequential accumulation in f32, as the C executor does
        acc = np.zeros([1 if d == axis else n for d, n in enumerate(a.shape)], dtype=f32)
        for i in range(a.shape[axis]):
            acc += np.take(a, [i], axis=axis)
        return acc
    if name in ("xt.matmul", "xt.mma"):
        out = np.asarray(vals[0], np.float64) @ np.asarray(vals[1], np.float64)
        if name == "xt.mma":
            out = out + np.asarray(vals[2], np.float64)
        return out.astype(f32)
    if name == "xt.reshape":
        return a.reshape(op.result_type.shape)
    if name == "xt.transpose":
        return np.ascontiguousarray(np.swapaxes(a, 1, 2))
    if name == "xt.permute":
        return np.ascontiguousarray(np.transpose(a, op.attrs["permutation"]))
    raise ValueError(f"interp: unsupported op {name}")
