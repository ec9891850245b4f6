"""GPU parity of seeded random matmul programs (tests/random_programs.py:
gemm_case): f16 / bf16 with an f32 result and the i8 epilogue form (A @ B *
scale + bias, rounded to i8), M, N, K multiples of 64 up to 1024 (K of 128 for
i8), Block tiles of 64, 128 or 256.

Bars: i8 bit-exact (exact i32 sums, the same f32 epilogue and rounding);
f16 / bf16 within a Frobenius relative error of 1e-3 of the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.gpu_util import frob_rel, run_gpu, run_oracle
from tests.random_programs import gemm_case, wide_gemm_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(40))
def test_random_gemm_matches_the_oracle(cuda, seed):
    mod, host, dtypes, out, desc = gemm_case(seed)
    assert xt.plan(mod)["kernel"].startswith("gemm")
    got = run_gpu(mod, host, dtypes, cuda, case=f"random gemm {seed}: {desc}")[out]
    want = run_oracle(mod, host, 8)[out]
    if dtypes[0] == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= 1e-3


@pytest.mark.parametrize("seed", range(30))
def test_random_wide_gemm_matches_the_oracle(cuda, seed):
    """M, N multiples of 128 up to 2048 (tests/random_programs.py:
    wide_gemm_case): the DMA kernel at every tile it chooses and the K split."""
    mod, host, dtypes, out, desc = wide_gemm_case(seed)
    assert xt.plan(mod)["kernel"].startswith("gemm")
    got = run_gpu(mod, host, dtypes, cuda, case=f"random wide gemm {seed}: {desc}")[out]
    want = run_oracle(mod, host, 8)[out]
    if dtypes[0] == "i8":
        assert np.array_equal(got, want)
    else:
        assert frob_rel(got, want) <= 1e-3
