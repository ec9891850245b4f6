"""GPU launches through the compiled ``_xtile`` module (xtile_amd/csrc/XTModule.cpp),
the stand-in for the reference's nanobind module (python/XTModule.cpp:210-231),
against the oracle and against the same launch through the ctypes binding.

One program per kernel family at a small size; bars as everywhere: bit-exact
for f32 add, relative error <= 1e-5 for softmax, Frobenius <= 1e-3 for f16
matmul and conv.  The launch goes on a side stream (the stream argument is a
hipStream_t as an integer)."""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.conftest import oracle_threads
from tests.gpu_util import frob_rel, run_oracle, to_device, to_host
from xtile_amd import kernels as K
from xtile_amd._compiled import load

pytestmark = pytest.mark.gpu


def _cases():
    rng = np.random.default_rng(2024)
    a = rng.uniform(-1, 1, (256, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (256, 512)).astype(np.float32)
    yield "add", K.add(256, 512), [a, b, np.zeros_like(a)], ["f32"] * 3, 2, "exact"
    x = rng.normal(0, 2, (64, 4096)).astype(np.float32)
    yield "softmax", K.softmax(64, 4096, 1), [x, np.zeros_like(x)], ["f32"] * 2, 1, "rel"
    pa = rng.uniform(-1, 1, (256, 512)).astype(np.float16)
    pb = rng.uniform(-1, 1, (512, 256)).astype(np.float16)
    yield ("matmul", K.matmul_f16(256, 256, 512, 128, 128), [pa, pb, np.zeros((256, 256), np.float32)],
           ["f16", "f16", "f32"], 2, "frob")
    ci = rng.normal(0, 0.5, (2, 8, 8, 64)).astype(np.float16)
    cf = rng.normal(0, 0.5, (3, 3, 64, 64)).astype(np.float16)
    yield ("conv", K.conv2d(2, 8, 8, 64, 64, 3, 3, 4, 8), [ci, cf, np.zeros((2, 8, 8, 64), np.float32)],
           ["f16", "f16", "f32"], 2, "frob")


@pytest.mark.parametrize("case", list(_cases()), ids=lambda c: c[0])
def test_compiled_module_launch(cuda, case):
    import torch

    name, module, host, dtypes, out, bar = case
    compiled = load()
    cap = compiled.parse(xt._wrap_module_asm(str(module))[0])
    desc, _, _ = compiled.plan(cap, None)
    assert desc == xt.plan(module)["kernel"]
    print(f"[gpu] compiled _xtile launch {name}: {desc}", flush=True)
    stream = torch.cuda.Stream(device=cuda)
    bufs = [to_device(h, d, cuda) for h, d in zip(host, dtypes)]
    twin = [t.clone() for t in bufs]
    torch.cuda.synchronize()
    compiled.launch(cap, None, [t.data_ptr() for t in bufs], [t.numel() * t.element_size() for t in bufs],
                    stream.cuda_stream)
    with torch.cuda.stream(stream):
        xt.launch(module, *twin, stream=stream)  # the ctypes binding
    torch.cuda.synchronize()
    got = to_host(bufs[out], dtypes[out])
    assert np.array_equal(got.view(np.uint32), to_host(twin[out], dtypes[out]).view(np.uint32))
    want = run_oracle(module, host, oracle_threads())[out]
    if bar == "exact":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    elif bar == "rel":
        assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
    else:
        assert frob_rel(got, want) <= 1e-3
