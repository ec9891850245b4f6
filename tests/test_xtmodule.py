"""The compiled ``_xtile`` module (xtile_amd/csrc/XTModule.cpp, pybind11) over
the C ABI, against the ctypes binding of the same ABI (xtile_amd/_xtile.py).

The compiled module stands in for the reference's nanobind ``_xtile``
(python/XTModule.cpp:210-231): it must carry that module's function and
keyword names, take a module capsule or any object with ``_CAPIPtr``
(XTModule.cpp:37-51), return the same object from a pass (runPass :128-151)
and raise the same exception types.  Every result is compared with the
ctypes binding's on the same text: the golden DSL programs (the reference
tracer's output), the benchmark configurations and seeded random programs.
Host only: no device is touched (launch is checked up to its buffer
refusals; tests/test_gpu_binding.py runs it).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

import xtile_amd as xt
from tests import random_programs as RP
from xtile_amd import _xtile as cbind
from xtile_amd import kernels as K
from xtile_amd._compiled import MODULE_PATH, load

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden" / "dsl"

compiled = load()

# python/XTModule.cpp:210-231
REFERENCE_NAMES = [
    "parse", "xt_to_nova", "xt_serialize", "nova_optimize", "nova_allocate",
    "nova_threading", "nova_barrier", "nova_to_x1", "_parse_module", "_module_asm",
]
BACKEND_NAMES = ["canonicalize", "func_names", "signature", "plan", "launch", "version"]


def _corpus() -> dict[str, str]:
    texts = {f"golden/{p.stem}": p.read_text() for p in sorted(GOLDEN.glob("*.mlir"))}
    for name, make in K.CONFIGS.items():
        texts[name] = str(make())
    texts["layernorm"] = str(K.layernorm(64, 256, 8))
    texts["column_softmax"] = str(K.column_softmax(64, 128, 32))
    texts["bias_add"] = str(K.bias_add(64, 128))
    texts["conv_strided_bf16"] = str(K.conv2d(2, 17, 19, 32, 32, 3, 3, 3, 10, dtype=K.bfloat16, stride=(2, 2)))
    for seed in range(12):
        texts[f"random/{seed}"] = RP.program(seed)[0]
    for seed in range(4):
        texts[f"random_fused/{seed}"] = RP.fused_program(seed)[0]
    return texts


CORPUS = _corpus()


def _outcome(fn, *args):
    """('ok', value) or (exception type, message)."""
    try:
        return "ok", fn(*args)
    except (ValueError, TypeError, RuntimeError, NotImplementedError) as e:
        return type(e), str(e)


def test_module_is_built_and_named_like_the_reference():
    assert MODULE_PATH.exists()
    assert compiled.__name__.endswith("_xtile")
    for name in REFERENCE_NAMES + BACKEND_NAMES:
        assert callable(getattr(compiled, name)), name
        assert callable(getattr(cbind, name)), name
    assert compiled.version() == cbind.version()


def test_reference_keyword_names():
    text = xt._wrap_module_asm(CORPUS["c1_add"])[0]
    cap = compiled.parse(asm=text)
    assert compiled._parse_module(asm=text) is not cap
    assert compiled.xt_serialize(module=cap) is cap
    assert "xt.store" in compiled._module_asm(module=cap)


@pytest.mark.parametrize("name", sorted(CORPUS))
def test_same_results_as_the_ctypes_binding(name):
    text = xt._wrap_module_asm(CORPUS[name])[0]
    a, b = cbind.parse(text), compiled.parse(text)
    assert type(b).__name__ == "PyCapsule"
    assert compiled._module_asm(b) == cbind._module_asm(a)
    funcs = compiled.func_names(b)
    assert funcs == cbind.func_names(a)
    for f in funcs:
        assert compiled.signature(b, f) == cbind.signature(a, f)
        assert _outcome(compiled.plan, b, f) == _outcome(cbind.plan, a, f)
    grid = compiled.signature(b, funcs[0])["grid"]
    passes = ["canonicalize", "xt_to_nova"]
    if grid[0] * grid[1] * grid[2] <= 256:  # serialize unrolls the grid
        passes.append("xt_serialize")
    for p in passes:
        a, b = cbind.parse(text), compiled.parse(text)
        ra, rb = _outcome(getattr(cbind, p), a), _outcome(getattr(compiled, p), b)
        assert ra[0] == rb[0], (p, ra, rb)
        if ra[0] == "ok":
            assert rb[1] is b
            assert compiled._module_asm(b) == cbind._module_asm(a), p
        else:
            assert ra[1] == rb[1], p


def test_errors_match_the_ctypes_binding():
    bad_text = "func.func @f( {"
    assert _outcome(compiled.parse, bad_text) == _outcome(cbind.parse, bad_text)
    assert _outcome(compiled.parse, bad_text)[0] is ValueError
    assert _outcome(compiled.parse, bad_text)[1].startswith("failed to parse test module\n")
    for wrong in (object(), "module {}", None, 7):
        for fn in ("_module_asm", "xt_serialize", "xt_to_nova", "canonicalize", "nova_optimize", "plan"):
            assert _outcome(getattr(compiled, fn), wrong) == (TypeError, "expected an xtile module object"), fn
    assert _outcome(compiled.parse, b"module {}") == (TypeError, "asm must be a str")
    assert _outcome(cbind.parse, b"module {}") == (TypeError, "asm must be a str")
    # a pass that fails: RuntimeError with the diagnostic text
    nogrid = compiled.parse("module {\n  func.func @f() {\n    func.return\n  }\n}")
    got = _outcome(compiled.xt_serialize, nogrid)
    assert got[0] is RuntimeError and "xt-serialize requires func.func xt.grid attribute" in got[1]
    assert got == _outcome(cbind.xt_serialize, cbind.parse("module {\n  func.func @f() {\n    func.return\n  }\n}"))
    # the x1 stages: NotImplementedError, same text
    cap = compiled.parse(xt._wrap_module_asm(CORPUS["c1_add"])[0])
    handle = cbind.parse(xt._wrap_module_asm(CORPUS["c1_add"])[0])
    for stage in ("nova_optimize", "nova_allocate", "nova_threading", "nova_barrier", "nova_to_x1"):
        got = _outcome(getattr(compiled, stage), cap)
        assert got[0] is NotImplementedError and stage in got[1]
        assert got == _outcome(getattr(cbind, stage), handle)
    # a program with no HIP kernel (its last tile overruns the array):
    # NotImplementedError from plan, same text
    overrun = xt._wrap_module_asm(str(K.add_rows(100, 128, 64)))[0]
    got = _outcome(compiled.plan, compiled.parse(overrun))
    assert got[0] is NotImplementedError and "exceeds extent" in got[1]
    assert got == _outcome(cbind.plan, cbind.parse(overrun))


def test_objects_with_capiptr_are_accepted():
    class Holder:
        def __init__(self, raw):
            self._CAPIPtr = raw

    cap = compiled.parse(xt._wrap_module_asm(CORPUS["bias_add"])[0])
    h = Holder(cap)
    assert compiled.xt_serialize(h) is h
    assert compiled._module_asm(h) == compiled._module_asm(cap)
    # a ctypes handle is not a capsule of this module
    assert _outcome(compiled._module_asm, Holder(cbind.parse("module {\n}"))) == (
        TypeError, "expected an xtile module object")


def test_capsules_free_their_modules():
    import gc

    text = xt._wrap_module_asm(CORPUS["c4_conv2d_f16"])[0]
    for _ in range(200):
        cap = compiled.parse(text)
        del cap
    gc.collect()
    cap = compiled.parse(text)
    assert compiled.func_names(cap) == ["conv2d_kernel"]


def test_launch_rejects_bad_buffers_before_any_device_call():
    cap = compiled.parse(xt._wrap_module_asm(str(K.add(64, 128)))[0])
    fake = [0x1000, 0x2000, 0x3000]
    with pytest.raises(ValueError, match="ptrs and sizes differ in length"):
        compiled.launch(cap, None, fake, [32768])
    with pytest.raises(ValueError, match="takes 3 buffers, got 2"):
        compiled.launch(cap, None, fake[:2], [32768, 32768])
    with pytest.raises(ValueError, match="needs 32768"):
        compiled.launch(cap, None, fake, [32768, 32768, 100])
    with pytest.raises(ValueError, match="is null"):
        compiled.launch(cap, None, [0x1000, 0, 0x3000], [32768] * 3)


FACADE_SCRIPT = """
import sys, xtile_amd as xt
from xtile_amd import kernels as K
print(type(xt._native).__name__, xt._native.__name__)
for make in (lambda: K.softmax(64, 256, 1), lambda: K.conv2d(2, 8, 8, 32, 32, 3, 3, 4, 8),
             lambda: K.layernorm(64, 256, 8)):
    m = make()
    print(repr(m)); print(xt.plan(m)); print(xt.signature(m))
    print(str(xt.xt_serialize(xt.parse(str(m)))))
    xt.xt_to_nova(m); print(str(m))
"""


def test_facade_runs_on_the_compiled_binding():
    """XTILE_AMD_BINDING=compiled makes the facade call the compiled module;
    everything it prints matches the default (ctypes) facade's output."""
    outs = {}
    for binding in ("ctypes", "compiled"):
        env = dict(os.environ, XTILE_AMD_BINDING=binding, PYTHONPATH=str(ROOT))
        p = subprocess.run([sys.executable, "-c", FACADE_SCRIPT], env=env, cwd=ROOT,
                           capture_output=True, text=True, timeout=300)
        assert p.returncode == 0, p.stderr
        outs[binding] = p.stdout.splitlines()
    assert outs["ctypes"][0] == "module xtile_amd._xtile"
    assert outs["compiled"][0] == "module xtile_amd.lib._xtile"
    assert outs["ctypes"][1:] == outs["compiled"][1:]
    assert len(outs["ctypes"]) > 20
