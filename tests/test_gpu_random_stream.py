"""GPU parity of seeded random programs of the two streaming families
(tests/random_programs.py: stream_case): f32 add over any tile that divides
the array (odd sizes, 1-wide tiles) and row softmax of 1-16 row tiles over
1-8192 columns.

Bars: add bit-exact (IEEE f32 add); softmax within 1e-5 relative to the
oracle per element.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.gpu_util import run_gpu, run_oracle
from tests.random_programs import stream_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(40))
def test_random_stream_program_matches_the_oracle(cuda, seed):
    mod, host, dtypes, out, desc = stream_case(seed)
    kernel = xt.plan(mod)["kernel"]
    assert kernel.startswith("ew_binary" if desc.startswith("add") else "row_softmax")
    got = run_gpu(mod, host, dtypes, cuda, case=f"random stream {seed}: {desc}")[out]
    want = run_oracle(mod, host, 8)[out]
    if desc.startswith("add"):
        assert np.array_equal(got, want)
    else:
        assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5


@pytest.mark.parametrize("fuse", ["1", "0"])
def test_long_rows_without_float4_alignment_leave_the_softmax_kernel(cuda, monkeypatch, fuse):
    """3798 columns (not a multiple of 4) exceed what the softmax kernel holds
    without float4 vectors: the planner sends the program to the fused
    kernel's ragged layout (or, with XTILE_AMD_FUSE=0, to the tile
    interpreter); both match the oracle."""
    from xtile_amd import kernels as K

    monkeypatch.setenv("XTILE_AMD_FUSE", fuse)
    mod = K.softmax(122, 3798, 2)
    assert xt.plan(mod)["kernel"].startswith("fused f32 tile=2x3798" if fuse == "1" else "tile_vm")
    x = np.random.default_rng(48).normal(0, 2, (122, 3798)).astype(np.float32)
    got = run_gpu(mod, [x, np.zeros_like(x)], ["f32"] * 2, cuda, case=f"softmax 122x3798 fuse={fuse}")[1]
    want = run_oracle(mod, [x, np.zeros_like(x)], 8)[1]
    assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
