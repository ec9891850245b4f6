"""GPU parity of seeded random `load_conv2d` programs (tests/random_programs.py:
conv_case): i8 / f16 / bf16, 1x1 to 5x5 filters, strides and dilations of 1 or
2, asymmetric pads, channel counts from 3 to 128, output tiles of every divisor
of the output, on whichever conv kernel the planner picks.

Bars: i8 bit-exact (exact i32 sums, one rounding to f32); f16 / bf16 within a
Frobenius relative error of 1e-3 of the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.gpu_util import frob_rel, run_gpu, run_oracle
from tests.random_programs import conv_case, image_conv_case, wide_conv_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(40))
def test_random_conv_matches_the_oracle(cuda, seed):
    mod, host, dtypes, desc = conv_case(seed)
    got = run_gpu(mod, host, dtypes, cuda, case=f"random conv {seed}: {desc}")[2]
    want = run_oracle(mod, host, 4)[2]
    if dtypes[0] == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= 1e-3


@pytest.mark.parametrize("seed", range(30))
def test_random_wide_conv_matches_the_oracle(cuda, seed):
    """Cin / Cout multiples of 8 (16 for i8) up to 320 / 256 over the whole
    output (tests/random_programs.py: wide_conv_case): the implicit-GEMM kernel
    wherever the band kernel declines."""
    mod, host, dtypes, desc = wide_conv_case(seed)
    got = run_gpu(mod, host, dtypes, cuda, case=f"random wide conv {seed}: {desc}")[2]
    want = run_oracle(mod, host, 8)[2]
    if dtypes[0] == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= 1e-3


@pytest.mark.parametrize("seed", range(16))
def test_random_resident_image_conv_matches_the_oracle(cuda, monkeypatch, seed):
    """Shapes in the resident-image kernel's range (tests/random_programs.py:
    image_conv_case), forced onto it with XTILE_AMD_CONV_IMAGE=1 whatever
    the image size and workgroup count: 1 x 3 to 5 x 3 filters, strides,
    dilations, asymmetric pads, 64 to 256 input and 32 to 256 output
    channels; every output is overwritten (the buffer starts at 7)."""
    monkeypatch.setenv("XTILE_AMD_CONV_IMAGE", "1")
    mod, host, dtypes, desc = image_conv_case(seed)
    got = run_gpu(mod, host, dtypes, cuda, case=f"random image conv {seed}: {desc}")[2]
    want = run_oracle(mod, [host[0], host[1], np.zeros_like(host[2])], 8)[2]
    assert frob_rel(got, want) <= 1e-3
