"""Helpers for GPU parity tests: numpy <-> device tensors, launch, oracle run."""

from __future__ import annotations

import sys

import numpy as np

import oracle


def to_device(arr: np.ndarray, dtype: str, device):
    import torch

    if dtype == "bf16":
        t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr))
    return t.to(device)


def to_host(t, dtype: str) -> np.ndarray:
    import torch

    t = t.detach().cpu()
    if dtype == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def run_gpu(module, host_buffers, dtypes, device, func=None, case: str = ""):
    """Copy buffers to the GPU, launch, synchronise, return host copies."""
    import torch

    import xtile_amd as xt

    print(f"[gpu] {case}: {xt.plan(module, func)['kernel']}", flush=True)
    sys.stdout.flush()
    dev = [to_device(b, d, device) for b, d in zip(host_buffers, dtypes)]
    xt.launch(module, *dev, func=func)
    torch.cuda.synchronize()
    return [to_host(t, d) for t, d in zip(dev, dtypes)]


def run_oracle(module, host_buffers, nthreads: int):
    bufs = [np.array(b, copy=True) for b in host_buffers]
    oracle.run(str(module), bufs, nthreads)
    return bufs


def frob_rel(x: np.ndarray, ref: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-300))
