"""TEST INFRASTRUCTURE - the parity oracle.  Not part of the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker.  The product path (xtile_amd) never
routes through it.

    from oracle import run
    run(xt_text, [a, b, out], nthreads=8)   # numpy buffers, outputs written in place

Components:
  xt_oracle.c    loop-lowered C executor (closed-form sharing rule, OpenMP over
                 independent blocks); the CPU baseline of bench.py
  interp.py      literal Python restatement of the serialized semantics
                 (z -> y -> x block order, shared-load reuse cache), used to pin
                 the C executor on small grids
  closed_form.py numpy float64 formulas (softmax, matmul, NHWC conv, halo slice)
  xt_reader.py   regex reader of xt text, independent of the product parser

bf16 buffers are numpy uint16 arrays of raw bf16 bits (numpy has no bf16).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .xt_reader import RFunc, read_function

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libxt_oracle.so"

ELEM = {"f32": 0, "f16": 1, "bf16": 2, "i8": 3}
NP_DTYPE = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i8": np.int8}

CODES = {
    "xt.load": 1,
    "xt.load_conv2d": 2,
    "xt.store": 3,
    "xt.add": 10,
    "xt.sub": 11,
    "xt.mul": 12,
    "xt.exp": 20,
    "xt.cos": 21,
    "xt.sin": 22,
    "xt.reciprocal": 23,
    "xt.rsqrt": 24,
    "xt.sigmoid": 25,
    "xt.tanh": 26,
    "xt.silu": 27,
    "xt.itof": 28,
    "xt.ftoi": 29,
    "xt.reduce_sum": 30,
    "xt.reduce_max": 31,
    "xt.matmul": 40,
    "xt.mma": 41,
    "xt.reshape": 50,
    "xt.transpose": 51,
    "xt.permute": 52,
}

MAXR = 4


class XoOp(ctypes.Structure):
    _fields_ = [
        ("code", ctypes.c_int),
        ("dst", ctypes.c_int),
        ("a", ctypes.c_int),
        ("b", ctypes.c_int),
        ("c", ctypes.c_int),
        ("arg", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("shape", ctypes.c_longlong * MAXR),
        ("coord_axis", ctypes.c_int * MAXR),
        ("coord_val", ctypes.c_longlong * MAXR),
        ("shared", ctypes.c_int),
        ("axis", ctypes.c_int),
        ("pad", ctypes.c_longlong * 4),
        ("stride", ctypes.c_longlong * 2),
        ("dil", ctypes.c_longlong * 2),
        ("perm", ctypes.c_int * MAXR),
    ]


class XoProg(ctypes.Structure):
    _fields_ = [
        ("nargs", ctypes.c_int),
        ("arg_elem", ctypes.c_int * 16),
        ("arg_rank", ctypes.c_int * 16),
        ("arg_shape", (ctypes.c_longlong * MAXR) * 16),
        ("nvals", ctypes.c_int),
        ("val_rank", ctypes.c_int * 64),
        ("val_shape", (ctypes.c_longlong * MAXR) * 64),
        ("nops", ctypes.c_int),
        ("ops", ctypes.POINTER(XoOp)),
        ("grid", ctypes.c_int * 3),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing; run `python -m oracle.build`")
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.xo_run.restype = ctypes.c_int
        _lib.xo_run.argtypes = [ctypes.POINTER(XoProg), ctypes.POINTER(ctypes.c_void_p), ctypes.c_int]
        _lib.xo_f16_to_f32.restype = ctypes.c_float
        _lib.xo_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.xo_f32_to_f16.restype = ctypes.c_uint16
        _lib.xo_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.xo_bf16_to_f32.restype = ctypes.c_float
        _lib.xo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.xo_f32_to_bf16.restype = ctypes.c_uint16
        _lib.xo_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.xo_max_threads.restype = ctypes.c_int
    return _lib


class Compiled:
    """An RFunc lowered to the C executor's op table."""

    def __init__(self, fn: RFunc) -> None:
        self.fn = fn
        self.arg_index = {name: k for k, (name, _) in enumerate(fn.args)}
        self.coords: dict[str, tuple[int, int]] = {}  # ssa -> (axis, value)
        self.slots: dict[str, int] = {}
        self.val_shapes: list[tuple[int, ...]] = []
        ops: list[XoOp] = []
        for op in fn.ops:
            if op.name == "xt.get_tile_block_id":
                for k, r in enumerate(op.results[:3]):
                    self.coords[r] = (k, 0)
                continue
            if op.name == "arith.constant":
                self.coords[op.results[0]] = (-1, int(op.attrs["value"]))
                continue
            if op.name not in CODES:
                raise ValueError(f"oracle: unsupported op {op.name}")
            o = XoOp()
            o.code = CODES[op.name]
            o.dst = o.a = o.b = o.c = o.arg = -1
            if op.name == "xt.load":
                o.arg = self.arg_index[op.operands[0]]
                self._tile(o, op.result_type.shape, op.operands[1:])
                o.shared = int(op.attrs.get("shared", 0))
                o.dst = self._slot(op.results[0], op.result_type.shape)
            elif op.name == "xt.store":
                o.a = self.slots[op.operands[0]]
                o.arg = self.arg_index[op.operands[1]]
                self._tile(o, op.operand_types[0].shape, op.operands[2:])
            elif op.name == "xt.load_conv2d":
                o.arg = self.arg_index[op.operands[0]]
                o.b = self.slots[op.operands[1]]
                self._tile(o, op.result_type.shape, op.operands[2:])
                for k, v in enumerate(op.attrs["pad"]):
                    o.pad[k] = v
                for k, v in enumerate(op.attrs["stride"]):
                    o.stride[k] = v
                for k, v in enumerate(op.attrs["dilation"]):
                    o.dil[k] = v
                o.dst = self._slot(op.results[0], op.result_type.shape)
            else:
                names = ["a", "b", "c"]
                for k, operand in enumerate(op.operands):
                    setattr(o, names[k], self.slots[operand])
                shape = op.result_type.shape
                o.rank = len(shape)
                for d, n in enumerate(shape):
                    o.shape[d] = n
                if "axis" in op.attrs:
                    ax = int(op.attrs["axis"])
                    o.axis = ax if ax >= 0 else ax + len(op.operand_types[0].shape)
                if "permutation" in op.attrs:
                    for d, v in enumerate(op.attrs["permutation"]):
                        o.perm[d] = v
                o.dst = self._slot(op.results[0], shape)
            ops.append(o)
        self.ops = (XoOp * max(1, len(ops)))(*ops)
        self.nops = len(ops)

    def _slot(self, name: str, shape) -> int:
        if len(self.val_shapes) >= 64:
            raise ValueError("oracle: too many values")
        self.slots[name] = len(self.val_shapes)
        self.val_shapes.append(tuple(shape))
        return self.slots[name]

    def _tile(self, o: XoOp, shape, coord_names) -> None:
        o.rank = len(shape)
        for d, n in enumerate(shape):
            o.shape[d] = n
        for d, c in enumerate(coord_names):
            axis, value = self.coords[c]
            o.coord_axis[d] = axis
            o.coord_val[d] = value

    def prog(self) -> XoProg:
        p = XoProg()
        p.nargs = len(self.fn.args)
        for k, (_, t) in enumerate(self.fn.args):
            p.arg_elem[k] = ELEM[t.dtype]
            p.arg_rank[k] = len(t.shape)
            for d, n in enumerate(t.shape):
                p.arg_shape[k][d] = n
        p.nvals = len(self.val_shapes)
        for v, s in enumerate(self.val_shapes):
            p.val_rank[v] = len(s)
            for d, n in enumerate(s):
                p.val_shape[v][d] = n
        p.nops = self.nops
        p.ops = ctypes.cast(self.ops, ctypes.POINTER(XoOp))
        for k in range(3):
            p.grid[k] = self.fn.grid[k]
        return p


def check_buffers(fn: RFunc, buffers) -> None:
    if len(buffers) != len(fn.args):
        raise ValueError(f"@{fn.name} takes {len(fn.args)} buffers, got {len(buffers)}")
    for k, ((_, t), b) in enumerate(zip(fn.args, buffers)):
        if b.dtype != NP_DTYPE[t.dtype] or tuple(b.shape) != t.shape or not b.flags.c_contiguous:
            raise ValueError(f"oracle buffer {k}: need {t.dtype}{t.shape} C-contiguous")


def run(text: str, buffers, nthreads: int = 1, func: str | None = None) -> None:
    """Execute every block of the xt function `text` over numpy `buffers`."""
    fn = read_function(text, func)
    check_buffers(fn, buffers)
    comp = Compiled(fn)
    prog = comp.prog()
    ptrs = (ctypes.c_void_p * len(buffers))(*[b.ctypes.data for b in buffers])
    if lib().xo_run(ctypes.byref(prog), ptrs, int(nthreads)) != 0:
        raise MemoryError("oracle: allocation failed")


def max_threads() -> int:
    return lib().xo_max_threads()


# -- bf16 helpers (numpy has no bf16) ------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
