"""xtile_amd: the xtile tile-programming DSL with an MI355X (gfx950) backend.

The public API mirrors the reference package's facade (xtile/__init__.py):
the DSL (``kernel, bid, load, load_conv2d, store, add, ... , convert``), the
module wrapper ``Module``, ``parse``, ``xt_serialize``, ``xt_to_nova``,
``compile``, ``save_ir``, ``save_compile_results`` and ``cdiv``.  Where the
reference lowers nova further to command text for its "x1" NPU (the
``nova_*`` stages, which raise here), this package plans and launches
hand-written HIP kernels: ``compile`` validates and plans the launch, and
``launch`` runs the program on the GPU over caller-owned device tensors.

Extensions over the reference API: ``float16`` / ``bfloat16`` dtypes,
``canonicalize``, ``plan``, ``signature`` and ``launch``.
"""

from __future__ import annotations

import os
from typing import Any

if os.environ.get("XTILE_AMD_BINDING", "ctypes") == "compiled":
    from ._compiled import load as _load_compiled

    _native = _load_compiled()  # csrc/XTModule.cpp, the compiled _xtile
else:
    from . import _xtile as _native  # ctypes over the same C ABI
from .dsl import (
    Array,
    DType,
    add,
    astype,
    bfloat16,
    bid,
    convert as _convert_impl,
    cos,
    exp,
    float16,
    float32,
    int8,
    kernel,
    load,
    load_conv2d,
    matmul,
    max,
    mma,
    mul,
    reciprocal,
    reshape,
    rsqrt,
    sigmoid,
    silu,
    sin,
    store,
    sub,
    sum,
    tanh,
    transpose,
)


def cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def _wrap_module_asm(asm: str) -> tuple[str, str | None]:
    """Bare `func.func` text is parsed inside `module { }` but displayed as given
    (xtile/__init__.py:74-83)."""
    stripped = asm.strip()
    if stripped.startswith("module"):
        return stripped, None
    body = "\n".join(f"  {line}" if line else line for line in stripped.splitlines())
    return f"module {{\n{body}\n}}", stripped


class Module:
    """A parsed xt module (owns its native IR, like the reference's capsule)."""

    def __init__(self, raw_module: Any, display_asm: str | None = None) -> None:
        self._raw_module = raw_module
        self._display_asm = display_asm

    @property
    def _CAPIPtr(self):
        return self._raw_module

    def __str__(self) -> str:
        if self._display_asm is not None:
            return self._display_asm
        return _native._module_asm(self)

    def __repr__(self) -> str:
        names = ", ".join("@" + n for n in _native.func_names(self))
        return f"<xtile_amd.Module {names}>"

    def _clear_display_override(self) -> None:
        self._display_asm = None


def parse(asm: str) -> Module:
    wrapped, display = _wrap_module_asm(asm)
    return Module(_native.parse(wrapped), display_asm=display)


def _after_pass(module: Any, result: Any) -> Any:
    if isinstance(module, Module):
        module._clear_display_override()
        return module
    return result


def xt_serialize(module: Any):
    """Unroll the grid (lib/xt/XTSerialize.cpp); mutates and returns `module`."""
    return _after_pass(module, _native.xt_serialize(module))


def canonicalize(module: Any):
    """Fold x+0 / x-0 and drop dead pure ops (lib/xt/XTOps.cpp:399-449)."""
    return _after_pass(module, _native.canonicalize(module))


def xt_to_nova(module: Any):
    """Lower xt ops to the nova dialect (lib/xt/XTToNova.cpp): tile offsets
    resolved to start indices, conv halo slices, unit affines; mutates and
    returns `module`.  An IR-level stage only: the HIP kernels launch from
    the xt form."""
    return _after_pass(module, _native.xt_to_nova(module))


def _x1_stage(name: str):
    native = getattr(_native, name)

    def stage(module: Any):
        """A stage of the reference's x1 NPU lowering: raises
        NotImplementedError (the MI355X backend runs HIP kernels instead)."""
        return native(module)

    stage.__name__ = name
    stage.__qualname__ = name
    return stage


nova_optimize = _x1_stage("nova_optimize")
nova_threading = _x1_stage("nova_threading")
nova_barrier = _x1_stage("nova_barrier")
nova_allocate = _x1_stage("nova_allocate")
nova_to_x1 = _x1_stage("nova_to_x1")


def plan(module: Any, func: str | None = None) -> dict:
    """The HIP launch chosen for `func`: kernel description, algorithmic
    bytes and FLOPs per launch.  Raises NotImplementedError for programs the
    backend has no kernel for."""
    desc, nbytes, nflops = _native.plan(module, func)
    return {"kernel": desc, "bytes": nbytes, "flops": nflops}


def signature(module: Any, func: str | None = None) -> dict:
    return _native.signature(module, func)


def compile(module: Any):
    """Verify and plan the HIP launch of every function; returns `module`.

    The reference's `compile` (xtile/__init__.py:160-168) lowers to x1 command
    text; here the product of compilation is a cached launch plan, and the IR
    is left as written so that `str(module)` still shows the xt program."""
    for name in _native.func_names(module):
        _native.plan(module, name)
    return module


_TORCH_DTYPES = None


def _torch_dtype(name: str):
    global _TORCH_DTYPES
    import torch

    if _TORCH_DTYPES is None:
        _TORCH_DTYPES = {
            "f32": torch.float32,
            "f16": torch.float16,
            "bf16": torch.bfloat16,
            "i8": torch.int8,
            "i32": torch.int32,
        }
    return _TORCH_DTYPES[name]


def launch(module: Any, *buffers, func: str | None = None, stream: Any = None) -> None:
    """Run `func` on the GPU.  `buffers` are torch tensors on one GPU, one per
    memref argument in argument order, contiguous, with the memref's dtype and
    shape.  Asynchronous on `stream` (default: torch's current stream)."""
    import torch

    sig = _native.signature(module, func)
    args = sig["args"]
    if len(buffers) != len(args):
        raise ValueError(f"@{sig['name']} takes {len(args)} buffers, got {len(buffers)}")
    device = None
    ptrs, sizes = [], []
    for k, (t, a) in enumerate(zip(buffers, args)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"buffer {k} must be a torch.Tensor")
        if not t.is_cuda:
            raise ValueError(f"buffer {k} is not on a GPU")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all buffers must be on the same GPU")
        if t.dtype != _torch_dtype(a["dtype"]):
            raise TypeError(f"buffer {k} has dtype {t.dtype}; expected {a['dtype']}")
        if tuple(t.shape) != tuple(a["shape"]):
            raise ValueError(f"buffer {k} has shape {tuple(t.shape)}; expected {tuple(a['shape'])}")
        if not t.is_contiguous():
            raise ValueError(f"buffer {k} must be contiguous")
        ptrs.append(t.data_ptr())
        sizes.append(t.numel() * t.element_size())
    with torch.cuda.device(device):
        s = stream if stream is not None else torch.cuda.current_stream(device)
        handle = s.cuda_stream if hasattr(s, "cuda_stream") else int(s)
        _native.launch(module, sig["name"], ptrs, sizes, handle)


def convert(kernel_fn, *, args, grid, double_buffering=False):
    return _convert_impl(
        kernel_fn,
        args=args,
        grid=grid,
        double_buffering=double_buffering,
        parse_module=parse,
    )


def save_ir(ir: object, save_path: str) -> None:
    with open(save_path, "wt") as f:
        f.write(str(ir))


def save_compile_results(ir: object, save_dir: str) -> None:
    """Write the xt program, its serialized form and the HIP launch plan.

    Stage files follow the reference's numbering (xtile/__init__.py:186-205)
    for the stages this backend has: 0_xt.mlir, then 1_hip_plan.txt (the
    kernel that `launch` would run), then 2_xt_serialize.mlir and
    3_xt_to_nova.mlir (both mutate `ir`, as in the reference)."""
    os.makedirs(save_dir, exist_ok=True)
    save_ir(ir, os.path.join(save_dir, "0_xt.mlir"))
    lines = []
    for name in _native.func_names(ir):
        try:
            desc, nbytes, nflops = _native.plan(ir, name)
            lines.append(f"@{name}: {desc} bytes={nbytes:.0f} flops={nflops:.0f}")
        except NotImplementedError as exc:
            lines.append(f"@{name}: no HIP kernel ({exc})")
    with open(os.path.join(save_dir, "1_hip_plan.txt"), "wt") as f:
        f.write("\n".join(lines) + "\n")
    ir = xt_serialize(ir)
    save_ir(ir, os.path.join(save_dir, "2_xt_serialize.mlir"))
    ir = xt_to_nova(ir)
    save_ir(ir, os.path.join(save_dir, "3_xt_to_nova.mlir"))
    print("compiled kernel ->", save_dir)


def _module_asm(module: Any) -> str:
    return _native._module_asm(module)


def _parse_module(asm: str) -> Module:
    return parse(asm)


__all__ = [
    "Array",
    "DType",
    "Module",
    "add",
    "astype",
    "bfloat16",
    "bid",
    "canonicalize",
    "cdiv",
    "compile",
    "convert",
    "cos",
    "exp",
    "float16",
    "float32",
    "int8",
    "kernel",
    "launch",
    "load",
    "load_conv2d",
    "matmul",
    "max",
    "mma",
    "mul",
    "nova_allocate",
    "nova_barrier",
    "nova_optimize",
    "nova_threading",
    "nova_to_x1",
    "parse",
    "plan",
    "reciprocal",
    "reshape",
    "rsqrt",
    "save_compile_results",
    "save_ir",
    "sigmoid",
    "signature",
    "silu",
    "sin",
    "store",
    "sub",
    "sum",
    "tanh",
    "transpose",
    "xt_serialize",
    "xt_to_nova",
]
