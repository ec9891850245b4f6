"""Tracing DSL: records one Block's tile program and emits `xt` dialect text.

The user-facing API mirrors the reference tracer (`xtile/dsl.py`): the same
function names, keyword arguments, validation rules and error types, and the
same textual `func.func` output, so that existing kernels and golden text keep
working.  The emitted text is consumed by the native `xt` parser of this
package (`xtile_amd/csrc/ir.cpp`).

Reference behaviour followed here (file:line into the reference tree):
  * dtypes `float32`/`int8`                       xtile/dsl.py:14-15
  * Array validation                              xtile/dsl.py:19-33
  * int kernel args become compile-time constants xtile/dsl.py:181-192
  * SSA naming stems and `%zero`/`%cN` constants  xtile/dsl.py:699-732
  * load / load_conv2d / store validation         xtile/dsl.py:225-313,469-488
  * binary broadcast rule (rhs dims 1), result = lhs shape   xtile/dsl.py:658-679,754-759
  * reductions keep the reduced dim at 1          xtile/dsl.py:622-644
  * `a / b` is `a * reciprocal(b)`                xtile/dsl.py:354-357
  * text format                                   xtile/dsl.py:490-620

Extension (not in the reference, documented as such): `float16` and
`bfloat16` dtypes.  Narrow-float `matmul` and `load_conv2d` produce a float32
result, mirroring the reference's int8 -> float32 rule (xtile/dsl.py:369-370).
"""

from __future__ import annotations

import inspect
from dataclasses import dataclass
from typing import Callable, Sequence


# ---------------------------------------------------------------------------
# dtypes and arrays
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class DType:
    name: str
    mlir_name: str


float32 = DType(name="float32", mlir_name="f32")
int8 = DType(name="int8", mlir_name="i8")
# Extension dtypes (MFMA input types on gfx950).
float16 = DType(name="float16", mlir_name="f16")
bfloat16 = DType(name="bfloat16", mlir_name="bf16")

_NARROW_FLOATS = (float16, bfloat16)


def _all_positive_ints(values: object) -> bool:
    return (
        isinstance(values, tuple)
        and len(values) > 0
        and all(isinstance(v, int) and v > 0 for v in values)
    )


@dataclass(frozen=True)
class Array:
    """A global-memory array argument: static shape plus element type."""

    shape: tuple[int, ...]
    dtype: DType

    def __post_init__(self) -> None:
        if not isinstance(self.shape, tuple) or not self.shape:
            raise TypeError("shape must be a non-empty tuple of integers")
        if not _all_positive_ints(self.shape):
            raise TypeError("shape must contain positive integers")
        if not isinstance(self.dtype, DType):
            raise TypeError("dtype must be an xtile dtype")

    @property
    def ndim(self) -> int:
        return len(self.shape)


def _memref_type(array: Array) -> str:
    return "memref<" + "x".join(map(str, array.shape)) + "x" + array.dtype.mlir_name + ">"


def _tensor_type(shape: Sequence[int], dtype: DType) -> str:
    return "tensor<" + "x".join(map(str, shape)) + "x" + dtype.mlir_name + ">"


# ---------------------------------------------------------------------------
# traced values
# ---------------------------------------------------------------------------


class KernelFunction:
    """A Python function marked with `@xt.kernel`."""

    def __init__(self, fn: Callable[..., object]) -> None:
        self.fn = fn
        self.__name__ = fn.__name__
        self.__doc__ = fn.__doc__
        self.__wrapped__ = fn


@dataclass(frozen=True)
class KernelArg:
    index: int
    python_name: str
    array: Array


@dataclass(frozen=True)
class ScalarArg:
    index: int
    python_name: str
    value: int


@dataclass(frozen=True)
class BlockId:
    dim: int


@dataclass(frozen=True)
class ConstantIndex:
    value: int


@dataclass(frozen=True)
class TensorValue:
    ssa_name: str
    shape: tuple[int, ...]
    dtype: DType

    def __sub__(self, other: object) -> "TensorValue":
        return sub(self, other)

    def __mul__(self, other: object) -> "TensorValue":
        return mul(self, other)

    def __add__(self, other: object) -> "TensorValue":
        return add(self, other)

    def __truediv__(self, other: object) -> "TensorValue":
        return truediv(self, other)


Coord = "BlockId | ConstantIndex"


# Each recorded operation renders its own line of `xt` text.  The renderer
# needs the final argument names, which are only known once tracing ends
# (they depend on how often each array is loaded and stored).


@dataclass(frozen=True)
class _Load:
    result: TensorValue
    array: KernelArg
    index: tuple
    shared: int | None

    def render(self, names: dict[int, str]) -> str:
        attr = f" {{shared = {self.shared} : i64}}" if self.shared in (1, 2) else ""
        coords = _coords_text(self.index)
        types = ", ".join([_memref_type(self.array.array)] + ["i32"] * len(self.index))
        return (
            f"{self.result.ssa_name} = xt.load(%{names[self.array.index]}, {coords}){attr}"
            f" : ({types}) -> {_tensor_type(self.result.shape, self.result.dtype)}"
        )


@dataclass(frozen=True)
class _LoadConv2D:
    result: TensorValue
    array: KernelArg
    filter: TensorValue
    index: tuple
    group: int
    pad: tuple[int, int, int, int]
    stride: tuple[int, int]
    dilation: tuple[int, int]

    def render(self, names: dict[int, str]) -> str:
        def arr(values: Sequence[int]) -> str:
            return "array<i64: " + ", ".join(map(str, values)) + ">"

        attrs = (
            f"{{dilation = {arr(self.dilation)}, group = {self.group} : i64, "
            f"pad = {arr(self.pad)}, stride = {arr(self.stride)}}}"
        )
        types = ", ".join(
            [
                _memref_type(self.array.array),
                _tensor_type(self.filter.shape, self.filter.dtype),
            ]
            + ["i32"] * len(self.index)
        )
        return (
            f"{self.result.ssa_name} = xt.load_conv2d(%{names[self.array.index]}, "
            f"{self.filter.ssa_name}, {_coords_text(self.index)}) {attrs} : ({types}) -> "
            f"{_tensor_type(self.result.shape, self.result.dtype)}"
        )


@dataclass(frozen=True)
class _Store:
    array: KernelArg
    index: tuple
    tile: TensorValue

    def render(self, names: dict[int, str]) -> str:
        types = ", ".join(
            [_tensor_type(self.tile.shape, self.tile.dtype), _memref_type(self.array.array)]
            + ["i32"] * len(self.index)
        )
        return (
            f"xt.store({self.tile.ssa_name}, %{names[self.array.index]}, "
            f"{_coords_text(self.index)}) : ({types}) -> ()"
        )


@dataclass(frozen=True)
class _Compute:
    """Any tensor -> tensor op: `%r = xt.op(%a[, %b[, %c]]) [{axis}] : types -> type`."""

    op_name: str
    result: TensorValue
    operands: tuple[TensorValue, ...]
    axis: int | None = None

    def render(self, names: dict[int, str]) -> str:
        attr = f" {{axis = {self.axis} : i64}}" if self.axis is not None else ""
        operand_names = ", ".join(v.ssa_name for v in self.operands)
        operand_types = ", ".join(_tensor_type(v.shape, v.dtype) for v in self.operands)
        return (
            f"{self.result.ssa_name} = {self.op_name}({operand_names}){attr} : "
            f"{operand_types} -> {_tensor_type(self.result.shape, self.result.dtype)}"
        )


def _coords_text(index: tuple) -> str:
    parts = []
    for item in index:
        if isinstance(item, BlockId):
            parts.append(f"%bid#{item.dim}")
        else:
            parts.append("%zero" if item.value == 0 else f"%c{item.value}")
    return ", ".join(parts)


# ---------------------------------------------------------------------------
# tracer
# ---------------------------------------------------------------------------


class TraceContext:
    """Symbolic execution of one Block of a kernel."""

    def __init__(
        self,
        kernel: KernelFunction,
        args: tuple,
        grid: tuple[int, int, int],
        double_buffering: bool,
    ) -> None:
        if not (isinstance(grid, tuple) and len(grid) == 3 and _all_positive_ints(grid)):
            raise ValueError("grid must be a 3-tuple of positive integers")
        params = list(inspect.signature(kernel.fn).parameters.values())
        if len(params) != len(args):
            raise ValueError("convert args must match the kernel signature")

        self.kernel_name = kernel.fn.__name__
        self.grid = grid
        self.double_buffering = double_buffering
        kernel_args: list[KernelArg | ScalarArg] = []
        for position, (param, value) in enumerate(zip(params, args)):
            if isinstance(value, Array):
                kernel_args.append(KernelArg(position, param.name, value))
            elif isinstance(value, int):
                kernel_args.append(ScalarArg(position, param.name, value))
            else:
                raise TypeError("convert args must be xt.Array values or integers")
        self.kernel_args = tuple(kernel_args)
        self.ops: list = []
        self.used_block_ids = False
        self.load_counts = [0] * len(kernel_args)
        self.store_counts = [0] * len(kernel_args)
        self._stem_counts: dict[str, int] = {}
        self._constants: dict[int, str] = {}

    # -- helpers ------------------------------------------------------------

    def trace_arguments(self) -> tuple:
        return tuple(a if isinstance(a, KernelArg) else a.value for a in self.kernel_args)

    def _fresh(self, stem: str) -> str:
        n = self._stem_counts.get(stem, 0) + 1
        self._stem_counts[stem] = n
        return f"%{stem}" if n == 1 else f"%{stem}{n}"

    def _value(self, stem: str, shape: tuple[int, ...], dtype: DType) -> TensorValue:
        return TensorValue(self._fresh(stem), tuple(shape), dtype)

    @staticmethod
    def _need_arg(array: object) -> None:
        if not isinstance(array, KernelArg):
            raise TypeError("xtile load/store expect kernel arguments")

    @staticmethod
    def _need_tensor(value: object) -> None:
        if not isinstance(value, TensorValue):
            raise TypeError("xtile operation expects a tensor value")

    @staticmethod
    def _need_shape(shape: object) -> None:
        if not _all_positive_ints(shape):
            raise TypeError("shape must be a tuple of positive integers")

    def _coords(self, index: object) -> tuple:
        if not isinstance(index, tuple) or not index:
            raise TypeError("index must be a non-empty tuple of values")
        out = []
        for item in index:
            if isinstance(item, BlockId):
                out.append(item)
            elif isinstance(item, int):
                if item not in self._constants:
                    self._constants[item] = "%zero" if item == 0 else self._fresh(f"c{item}")
                out.append(ConstantIndex(item))
            else:
                raise TypeError("index values must be xt.bid(...) results or integers")
        return tuple(out)

    @staticmethod
    def _int_tuple(name: str, value: object, length: int, positive: bool = False) -> None:
        if not isinstance(value, tuple) or len(value) != length:
            raise TypeError(f"{name} must be a tuple of {length} integers")
        for item in value:
            if not isinstance(item, int):
                raise TypeError(f"{name} must be a tuple of {length} integers")
            if positive and item <= 0:
                raise ValueError(f"{name} values must be positive")
            if not positive and item < 0:
                raise ValueError(f"{name} values must be non-negative")

    # -- block ids, loads and stores -----------------------------------------

    def bid(self, dim: int) -> BlockId:
        if dim not in (0, 1, 2):
            raise ValueError("xt.bid only supports dimensions 0, 1, and 2")
        self.used_block_ids = True
        return BlockId(dim)

    def load(self, array, index, shape, shared=None) -> TensorValue:
        self._need_arg(array)
        coords = self._coords(index)
        self._need_shape(shape)
        if shared is not None and shared not in (0, 1, 2):
            raise ValueError("shared must be 0, 1, 2, or None")
        rank = array.array.ndim
        if rank != len(shape):
            raise ValueError("xt.load requires shape rank to match the source array rank")
        if len(coords) != len(shape):
            raise ValueError("xt.load requires index rank to match the source array rank")
        result = self._value("x", shape, array.array.dtype)
        self.ops.append(_Load(result, array, coords, shared))
        self.load_counts[array.index] += 1
        return result

    def load_conv2d(self, array, filter_value, index, shape, *, group=1, pad, stride, dilation):
        self._need_arg(array)
        self._need_tensor(filter_value)
        coords = self._coords(index)
        self._need_shape(shape)
        self._int_tuple("pad", pad, 4)
        self._int_tuple("stride", stride, 2, positive=True)
        self._int_tuple("dilation", dilation, 2, positive=True)
        if group <= 0:
            raise ValueError("xt.load_conv2d requires group to be positive")
        if array.array.ndim != 4:
            raise ValueError("xt.load_conv2d requires a rank-4 source memref")
        if len(filter_value.shape) != 4:
            raise ValueError("xt.load_conv2d requires a rank-4 filter tensor")
        if len(coords) != 4 or len(shape) != 4:
            raise ValueError("xt.load_conv2d requires rank-4 index and result shape tuples")
        src_dtype = array.array.dtype
        if src_dtype != filter_value.dtype or src_dtype not in (int8, *_NARROW_FLOATS):
            raise TypeError(
                "xt.load_conv2d requires int8, float16 or bfloat16 source/filter of one dtype"
            )
        if array.array.shape[3] != filter_value.shape[2]:
            raise ValueError("xt.load_conv2d requires source/filter channel dimensions to match")
        if shape[3] > filter_value.shape[3]:
            raise ValueError(
                "xt.load_conv2d result channel dimension must not exceed filter output channels"
            )
        result = self._value("load_conv", shape, float32)
        self.ops.append(
            _LoadConv2D(result, array, filter_value, coords, group, pad, stride, dilation)
        )
        self.load_counts[array.index] += 1
        return result

    def store(self, array, index, tile) -> None:
        self._need_arg(array)
        coords = self._coords(index)
        if not isinstance(tile, TensorValue):
            raise TypeError("xt.store expects a tensor value")
        if array.array.ndim != len(tile.shape):
            raise ValueError("xt.store requires tile rank to match the destination array rank")
        if len(coords) != len(tile.shape):
            raise ValueError("xt.store requires index rank to match the destination array rank")
        self.ops.append(_Store(array, coords, tile))
        self.store_counts[array.index] += 1

    # -- compute ----------------------------------------------------------

    def _unary(self, op_name: str, value, stem: str) -> TensorValue:
        self._need_tensor(value)
        result = self._value(stem, value.shape, value.dtype)
        self.ops.append(_Compute(op_name, result, (value,)))
        return result

    def _binary(self, op_name: str, lhs, rhs, stem: str) -> TensorValue:
        self._need_tensor(lhs)
        self._need_tensor(rhs)
        if lhs.dtype != rhs.dtype:
            raise TypeError("binary xtile ops require matching dtypes")
        same_rank = len(lhs.shape) == len(rhs.shape)
        if lhs.shape != rhs.shape and not (
            same_rank and all(r in (1, l) for l, r in zip(lhs.shape, rhs.shape))
        ):
            raise ValueError(
                "binary xtile ops require equal or rowwise-broadcast-compatible shapes"
            )
        result = self._value(stem, lhs.shape, lhs.dtype)
        self.ops.append(_Compute(op_name, result, (lhs, rhs)))
        return result

    def _reduce(self, op_name: str, value, stem: str, axis: int) -> TensorValue:
        self._need_tensor(value)
        if len(value.shape) != 2:
            raise ValueError("xt.max and xt.sum currently support rank-2 tensors only")
        if not isinstance(axis, int):
            raise TypeError("axis must be an integer")
        rank = len(value.shape)
        if not -rank <= axis < rank:
            raise ValueError("axis must be in range [-rank, rank)")
        axis %= rank
        shape = tuple(1 if d == axis else n for d, n in enumerate(value.shape))
        result = self._value(stem, shape, value.dtype)
        self.ops.append(_Compute(op_name, result, (value,), axis=axis))
        return result

    def reduce_max(self, value, axis: int = -1) -> TensorValue:
        return self._reduce("xt.reduce_max", value, "row_max", axis)

    def reduce_sum(self, value, axis: int = -1) -> TensorValue:
        return self._reduce("xt.reduce_sum", value, "row_sum", axis)

    def add(self, lhs, rhs):
        return self._binary("xt.add", lhs, rhs, "sum")

    def sub(self, lhs, rhs):
        return self._binary("xt.sub", lhs, rhs, "shifted")

    def mul(self, lhs, rhs):
        return self._binary("xt.mul", lhs, rhs, "normalized")

    def truediv(self, lhs, rhs):
        self._need_tensor(lhs)
        self._need_tensor(rhs)
        return self.mul(lhs, self.reciprocal(rhs))

    def exp(self, v):
        return self._unary("xt.exp", v, "exp")

    def cos(self, v):
        return self._unary("xt.cos", v, "cos")

    def sin(self, v):
        return self._unary("xt.sin", v, "sin")

    def reciprocal(self, v):
        return self._unary("xt.reciprocal", v, "inv_sum")

    def rsqrt(self, v):
        return self._unary("xt.rsqrt", v, "rsqrt")

    def sigmoid(self, v):
        return self._unary("xt.sigmoid", v, "sigmoid")

    def tanh(self, v):
        return self._unary("xt.tanh", v, "tanh")

    def silu(self, v):
        return self._unary("xt.silu", v, "silu")

    def matmul(self, lhs, rhs) -> TensorValue:
        self._need_tensor(lhs)
        self._need_tensor(rhs)
        if len(lhs.shape) != 2 or len(rhs.shape) != 2:
            raise ValueError("xt.matmul currently supports rank-2 tensors only")
        if lhs.shape[1] != rhs.shape[0]:
            raise ValueError("xt.matmul requires lhs inner dimension to match rhs outer dimension")
        if lhs.dtype == rhs.dtype and lhs.dtype in (int8, *_NARROW_FLOATS):
            out_dtype = float32
        elif lhs.dtype == rhs.dtype:
            out_dtype = lhs.dtype
        else:
            raise TypeError("xt.matmul requires matching dtypes or int8 inputs")
        result = self._value("matmul", (lhs.shape[0], rhs.shape[1]), out_dtype)
        self.ops.append(_Compute("xt.matmul", result, (lhs, rhs)))
        return result

    def mma(self, lhs, rhs, acc) -> TensorValue:
        for v in (lhs, rhs, acc):
            self._need_tensor(v)
        if len(lhs.shape) != 2 or len(rhs.shape) != 2 or len(acc.shape) != 2:
            raise ValueError("xt.mma currently supports rank-2 tensors only")
        if lhs.dtype != int8 or rhs.dtype != int8:
            raise TypeError("xt.mma requires int8 lhs and rhs tensors")
        if acc.dtype != float32:
            raise TypeError("xt.mma currently requires a float32 accumulator")
        if lhs.shape[1] != rhs.shape[0]:
            raise ValueError("xt.mma requires lhs inner dimension to match rhs outer dimension")
        if acc.shape != (lhs.shape[0], rhs.shape[1]):
            raise ValueError("xt.mma accumulator shape must match the matmul result shape")
        result = self._value("mma", acc.shape, acc.dtype)
        self.ops.append(_Compute("xt.mma", result, (lhs, rhs, acc)))
        return result

    def astype(self, value, dtype) -> TensorValue:
        self._need_tensor(value)
        if not isinstance(dtype, DType):
            raise TypeError("xt.astype requires an xtile dtype")
        if value.dtype == dtype:
            return value
        if value.dtype == int8 and dtype == float32:
            op_name = "xt.itof"
        elif value.dtype == float32 and dtype == int8:
            op_name = "xt.ftoi"
        else:
            raise TypeError("xt.astype only supports int8<->float32 conversions")
        result = self._value("cast", value.shape, dtype)
        self.ops.append(_Compute(op_name, result, (value,)))
        return result

    def reshape(self, value, shape) -> TensorValue:
        self._need_tensor(value)
        self._need_shape(shape)
        if _numel(value.shape) != _numel(shape):
            raise ValueError("xt.reshape requires the same number of elements")
        result = self._value("reshape", shape, value.dtype)
        self.ops.append(_Compute("xt.reshape", result, (value,)))
        return result

    def transpose(self, value) -> TensorValue:
        self._need_tensor(value)
        if len(value.shape) != 3:
            raise ValueError("xt.transpose currently supports rank-3 tensors only")
        b, m, n = value.shape
        result = self._value("transpose", (b, n, m), value.dtype)
        self.ops.append(_Compute("xt.transpose", result, (value,)))
        return result

    # -- emission ---------------------------------------------------------

    def _arg_names(self) -> dict[int, str]:
        """Loaded-only arrays are input/inputN, stored-only output/outputN."""
        names: dict[int, str] = {}
        n_in = n_out = 0
        for arg in self.kernel_args:
            if not isinstance(arg, KernelArg):
                continue
            loads, stores = self.load_counts[arg.index], self.store_counts[arg.index]
            if loads and not stores:
                n_in += 1
                names[arg.index] = "input" if n_in == 1 else f"input{n_in}"
            elif stores and not loads:
                n_out += 1
                names[arg.index] = "output" if n_out == 1 else f"output{n_out}"
            else:
                names[arg.index] = arg.python_name
        return names

    def emit_function_asm(self) -> str:
        names = self._arg_names()
        params = ", ".join(
            f"%{names[a.index]}: {_memref_type(a.array)}"
            for a in self.kernel_args
            if isinstance(a, KernelArg)
        )
        attrs = ["xt.grid = array<i32: " + ", ".join(map(str, self.grid)) + ">"]
        if self.double_buffering:
            attrs.append("xt.double_buffering = 1 : i32")
        out = [f"func.func @{self.kernel_name}({params}) attributes {{{', '.join(attrs)}}} {{"]
        if self.used_block_ids:
            out.append("  %bid:3 = xt.get_tile_block_id : i32, i32, i32")
        if self._constants:
            out.extend(
                f"  {name} = arith.constant {value} : i32"
                for value, name in sorted(self._constants.items())
            )
            out.append("")
        out.extend("  " + op.render(names) for op in self.ops)
        out.append("  func.return")
        out.append("}")
        return "\n".join(out)


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


# ---------------------------------------------------------------------------
# module-level API (valid only while a kernel is being converted)
# ---------------------------------------------------------------------------

_ACTIVE_TRACE: TraceContext | None = None


def _trace(what: str) -> TraceContext:
    if _ACTIVE_TRACE is None:
        raise RuntimeError(f"xt.{what} may only be used while converting a kernel")
    return _ACTIVE_TRACE


def kernel(fn: Callable[..., object]) -> KernelFunction:
    return KernelFunction(fn)


def bid(dim: int) -> BlockId:
    return _trace("bid").bid(dim)


def load(array, *, index, shape, shared=None) -> TensorValue:
    return _trace("load").load(array, index, shape, shared)


def load_conv2d(array, filter_value, *, index, shape, group=1, pad, stride, dilation):
    return _trace("load_conv2d").load_conv2d(
        array, filter_value, index, shape, group=group, pad=pad, stride=stride, dilation=dilation
    )


def store(array, *, index, tile) -> None:
    _trace("store").store(array, index, tile)


def max(input_value, axis: int = -1):  # noqa: A001 - mirrors the reference name
    return _trace("max").reduce_max(input_value, axis=axis)


def sum(input_value, axis: int = -1):  # noqa: A001 - mirrors the reference name
    return _trace("sum").reduce_sum(input_value, axis=axis)


def sub(lhs, rhs):
    return _trace("sub").sub(lhs, rhs)


def add(lhs, rhs):
    return _trace("add").add(lhs, rhs)


def mul(lhs, rhs):
    return _trace("mul").mul(lhs, rhs)


def truediv(lhs, rhs):
    ctx = _trace("truediv")
    if not isinstance(rhs, TensorValue):
        raise TypeError("xt.truediv currently requires a tensor rhs")
    return ctx.truediv(lhs, rhs)


def exp(v):
    return _trace("exp").exp(v)


def cos(v):
    return _trace("cos").cos(v)


def sin(v):
    return _trace("sin").sin(v)


def reciprocal(v):
    return _trace("reciprocal").reciprocal(v)


def rsqrt(v):
    return _trace("rsqrt").rsqrt(v)


def sigmoid(v):
    return _trace("sigmoid").sigmoid(v)


def tanh(v):
    return _trace("tanh").tanh(v)


def silu(v):
    return _trace("silu").silu(v)


def matmul(lhs, rhs):
    return _trace("matmul").matmul(lhs, rhs)


def mma(lhs, rhs, acc):
    return _trace("mma").mma(lhs, rhs, acc)


def astype(input_value, *, dtype):
    return _trace("astype").astype(input_value, dtype)


def reshape(input_value, *, shape):
    return _trace("reshape").reshape(input_value, shape)


def transpose(input_value):
    return _trace("transpose").transpose(input_value)


def convert(kernel_fn, *, args, grid, double_buffering, parse_module):
    """Trace `kernel_fn` once and hand the emitted text to `parse_module`."""
    global _ACTIVE_TRACE
    if not isinstance(kernel_fn, KernelFunction):
        raise TypeError("xt.convert expects a function decorated with @xt.kernel")
    trace = TraceContext(kernel_fn, args, grid, double_buffering)
    outer = _ACTIVE_TRACE
    _ACTIVE_TRACE = trace
    try:
        returned = kernel_fn.fn(*trace.trace_arguments())
    finally:
        _ACTIVE_TRACE = outer
    if returned is not None:
        raise ValueError("xt.kernel functions must not return a value")
    return parse_module(trace.emit_function_asm())
