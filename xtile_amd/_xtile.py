"""ctypes binding of ``libxtile_amd.so`` (C ABI: ``include/xtile_amd.h``).

Presents the functions of the reference's nanobind module ``_xtile``
(python/XTModule.cpp:210-231) with the same names, argument meaning and
exception types:

  parse(asm) / _parse_module(asm)   ValueError("failed to parse test module")
  xt_serialize(module)              returns the same object, RuntimeError on failure
  _module_asm(module)               str
  TypeError for objects that are not xtile modules (XTModule.cpp:40-51)

and ``nova_optimize`` / ``nova_threading`` / ``nova_barrier`` /
``nova_allocate`` / ``nova_to_x1``, which raise NotImplementedError (there is
no x1 NPU target), plus what the GPU backend adds: ``canonicalize``,
``xt_to_nova``, ``signature``, ``plan`` and ``launch``.  The library is loaded from ``xtile_amd/lib``; if it is missing the
import fails loudly - there is no fallback path.
"""

from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "lib" / "libxtile_amd.so"

XT_OK = 0
XT_ERR_PARSE = 1
XT_ERR_TYPE = 2
XT_ERR_PASS = 3
XT_ERR_UNSUPPORTED = 4
XT_ERR_ARGUMENT = 5
XT_ERR_DEVICE = 6

# Every symbol include/xtile_amd.h declares, with its ctypes signature.
_c_char_pp = ctypes.POINTER(ctypes.c_char_p)
SIGNATURES = {
    "xt_free": (None, [ctypes.c_void_p]),
    "xt_version": (ctypes.c_char_p, []),
    "xt_module_parse": (
        ctypes.c_int,
        [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)],
    ),
    "xt_module_free": (None, [ctypes.c_void_p]),
    "xt_module_print": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)],
    ),
    "xt_pass_run": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "xt_module_num_funcs": (ctypes.c_int, [ctypes.c_void_p]),
    "xt_module_func_name": (ctypes.c_char_p, [ctypes.c_void_p, ctypes.c_int]),
    "xt_func_signature": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)],
    ),
    "xt_plan": (
        ctypes.c_int,
        [
            ctypes.c_void_p,
            ctypes.c_char_p,
            ctypes.POINTER(ctypes.c_void_p),
            ctypes.POINTER(ctypes.c_double),
            ctypes.POINTER(ctypes.c_double),
            ctypes.POINTER(ctypes.c_void_p),
        ],
    ),
    "xt_gpu_run": (
        ctypes.c_int,
        [
            ctypes.c_void_p,
            ctypes.c_char_p,
            ctypes.POINTER(ctypes.c_void_p),
            ctypes.POINTER(ctypes.c_size_t),
            ctypes.c_int,
            ctypes.c_void_p,
            ctypes.POINTER(ctypes.c_void_p),
        ],
    ),
}


def _load() -> ctypes.CDLL:
    path = os.environ.get("XTILE_AMD_LIB", str(_LIB_PATH))
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built; run `python xtile_amd/build.py` (or __graft_entry__.build())"
        )
    # One HIP runtime per process.  PyTorch-ROCm ships its own libamdhip64 /
    # libhsa-runtime64 (loaded under file names without the .7 / .1 suffix but
    # with the same SONAMEs).  Importing torch first makes its runtime the one
    # our library's NEEDED entries bind to; loading ours first would map a
    # second runtime that then finds no device once torch owns it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = _load()
LIB_FILE = os.environ.get("XTILE_AMD_LIB", str(_LIB_PATH))


def _take_string(ptr: ctypes.c_void_p) -> str:
    if not ptr.value:
        return ""
    try:
        return ctypes.string_at(ptr.value).decode()
    finally:
        lib.xt_free(ptr)


class NativeModule:
    """Owning handle of one parsed module (the reference's PyCapsule)."""

    __slots__ = ("_ptr",)

    def __init__(self, ptr: int) -> None:
        self._ptr = ptr

    @property
    def ptr(self) -> int:
        return self._ptr

    def __del__(self) -> None:
        ptr, self._ptr = getattr(self, "_ptr", None), None
        if ptr and lib is not None:
            lib.xt_module_free(ptr)


def _unwrap(module: object) -> NativeModule:
    if isinstance(module, NativeModule):
        return module
    raw = getattr(module, "_CAPIPtr", None)
    if isinstance(raw, NativeModule):
        return raw
    raise TypeError("expected an xtile module object")


def _raise(status: int, message: str, default: str) -> None:
    text = message or default
    if status == XT_ERR_PARSE:
        raise ValueError("failed to parse test module" + (f"\n{message}" if message else ""))
    if status == XT_ERR_TYPE:
        raise TypeError(text)
    if status == XT_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    if status == XT_ERR_ARGUMENT:
        raise ValueError(text)
    raise RuntimeError(text)


def parse(asm: str) -> NativeModule:
    if not isinstance(asm, str):
        raise TypeError("asm must be a str")
    data = asm.encode()
    out = ctypes.c_void_p()
    err = ctypes.c_void_p()
    st = lib.xt_module_parse(data, len(data), ctypes.byref(out), ctypes.byref(err))
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, "failed to parse test module")
    return NativeModule(out.value)


_parse_module = parse


def _run_pass(module: object, name: str) -> object:
    handle = _unwrap(module)
    err = ctypes.c_void_p()
    st = lib.xt_pass_run(handle.ptr, name.encode(), ctypes.byref(err))
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, f"xtile.{name.replace('-', '_')} failed")
    return module


def xt_serialize(module: object) -> object:
    return _run_pass(module, "xt-serialize")


def canonicalize(module: object) -> object:
    return _run_pass(module, "canonicalize")


def xt_to_nova(module: object) -> object:
    return _run_pass(module, "xt-to-nova")


def _x1_stage(name: str):
    """The reference module's NPU lowering stages (python/XTModule.cpp:
    nova_optimize, nova_threading, nova_barrier, nova_allocate, nova_to_x1),
    which the reference facade calls from compile and save_compile_results
    (xtile/__init__.py:130-168).  The HIP backend has no x1 NPU target, so
    each checks its argument as the reference's runPass does (TypeError for a
    non-module) and then raises NotImplementedError naming what to use."""

    def stage(module: object) -> object:
        _unwrap(module)
        raise NotImplementedError(
            f"{name} belongs to the reference's x1 NPU lowering, which the MI355X "
            "backend replaces with HIP kernels; use xt.compile / xt.launch"
        )

    stage.__name__ = name
    stage.__qualname__ = name
    return stage


nova_optimize = _x1_stage("nova_optimize")
nova_threading = _x1_stage("nova_threading")
nova_barrier = _x1_stage("nova_barrier")
nova_allocate = _x1_stage("nova_allocate")
nova_to_x1 = _x1_stage("nova_to_x1")


def _module_asm(module: object) -> str:
    handle = _unwrap(module)
    out = ctypes.c_void_p()
    err = ctypes.c_void_p()
    st = lib.xt_module_print(handle.ptr, ctypes.byref(out), ctypes.byref(err))
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, "printing failed")
    return _take_string(out)


def func_names(module: object) -> list[str]:
    handle = _unwrap(module)
    n = lib.xt_module_num_funcs(handle.ptr)
    return [lib.xt_module_func_name(handle.ptr, k).decode() for k in range(n)]


def signature(module: object, func: str | None = None) -> dict:
    handle = _unwrap(module)
    out = ctypes.c_void_p()
    err = ctypes.c_void_p()
    st = lib.xt_func_signature(
        handle.ptr, (func or "").encode(), ctypes.byref(out), ctypes.byref(err)
    )
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, "signature failed")
    return json.loads(_take_string(out))


def plan(module: object, func: str | None = None) -> tuple[str, float, float]:
    """(kernel description, algorithmic bytes, algorithmic FLOPs) of one launch."""
    handle = _unwrap(module)
    out = ctypes.c_void_p()
    err = ctypes.c_void_p()
    nbytes = ctypes.c_double()
    nflops = ctypes.c_double()
    st = lib.xt_plan(
        handle.ptr,
        (func or "").encode(),
        ctypes.byref(out),
        ctypes.byref(nbytes),
        ctypes.byref(nflops),
        ctypes.byref(err),
    )
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, "planning failed")
    return _take_string(out), nbytes.value, nflops.value


def launch(module: object, func: str | None, ptrs, sizes, stream: int = 0) -> None:
    """Enqueue `func` on `stream` with device pointers `ptrs` (memref order)."""
    handle = _unwrap(module)
    n = len(ptrs)
    if len(sizes) != n:
        raise ValueError("ptrs and sizes differ in length")
    arr_p = (ctypes.c_void_p * n)(*ptrs)
    arr_s = (ctypes.c_size_t * n)(*sizes)
    err = ctypes.c_void_p()
    st = lib.xt_gpu_run(
        handle.ptr,
        (func or "").encode(),
        arr_p,
        arr_s,
        n,
        ctypes.c_void_p(stream or None),
        ctypes.byref(err),
    )
    msg = _take_string(err)
    if st != XT_OK:
        _raise(st, msg, "launch failed")


def version() -> str:
    return lib.xt_version().decode()
