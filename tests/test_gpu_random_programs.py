"""GPU parity of seeded random tile programs (tests/random_programs.py):
loads of every element type, broadcast add / sub / mul, bounded unary ops,
keep-dim reductions, transposes and matmuls (on the fused kernel when the
program fits its form, else on the tile interpreter), and programs generated in
the fused kernel's form at sizes up to 6000 Blocks.

Bars: narrow (f16 / bf16) stores of add / sub / mul results are bit-exact
(the same f32 operations, then the same rounding); the f32 output within
rtol 2e-5 plus 2e-5 of its largest magnitude (device libm against glibc for
the transcendental ops, other summation orders for reductions and matmul).
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from oracle import bf16_bits_to_f32
from tests.gpu_util import run_gpu, run_oracle
from tests.random_programs import program

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(60))
def test_random_program_matches_the_oracle(cuda, seed):
    text, host, dtypes, out = program(seed)
    m = xt.parse(text)
    got = run_gpu(m, host, dtypes, cuda, case=f"random program {seed}")
    want = run_oracle(m, host, 1)
    for k, d in enumerate(dtypes):
        if k == out:
            w = want[k].astype(np.float64)
            np.testing.assert_allclose(got[k], w, rtol=2e-5, atol=2e-5 * max(1.0, np.abs(w).max()))
        elif d in ("f16", "bf16") and not np.array_equal(host[k], want[k]):  # a stored narrow tile
            assert np.array_equal(got[k].view(np.uint16), want[k].view(np.uint16))
        else:  # inputs are not written
            assert np.array_equal(got[k], host[k])


@pytest.mark.parametrize("seed", range(40))
def test_fusable_random_program_matches_the_oracle(cuda, seed):
    """Programs of the fused kernel's form (tests/random_programs.py:
    fused_program), up to 6000 Blocks; same bars as above."""
    from tests.random_programs import fused_program

    text, host, dtypes, outs = fused_program(seed)
    m = xt.parse(text)
    assert xt.plan(m)["kernel"].startswith("fused")
    got = run_gpu(m, host, dtypes, cuda, case=f"fusable random program {seed}")
    want = run_oracle(m, host, 4)
    for k, d in enumerate(dtypes):
        if k in outs:
            w = want[k].astype(np.float64)
            np.testing.assert_allclose(got[k], w, rtol=2e-5, atol=2e-5 * max(1.0, np.abs(w).max()))
        elif d in ("f16", "bf16") and not np.array_equal(host[k], want[k]):
            assert np.array_equal(got[k].view(np.uint16), want[k].view(np.uint16))
        else:
            assert np.array_equal(got[k], host[k])
