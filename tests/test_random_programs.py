"""Seeded random tile programs (tests/random_programs.py): every one plans
onto a HIP kernel and runs in the oracle (CPU); on the GPU every one matches
the oracle (test_gpu_random_programs.py)."""

from __future__ import annotations

import pytest

import xtile_amd as xt
from tests.gpu_util import run_oracle
from tests.random_programs import program

SEEDS = range(60)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_plans_and_runs_in_the_oracle(seed):
    text, host, dtypes, out = program(seed)
    m = xt.parse(text)
    assert xt.plan(m)["kernel"]
    got = run_oracle(m, host, 1)
    assert got[out].shape == host[out].shape


@pytest.mark.parametrize("seed", range(40))
def test_fusable_random_program_plans_onto_a_fused_kernel(seed):
    from tests.random_programs import fused_program

    text, host, dtypes, outs = fused_program(seed)
    assert xt.plan(xt.parse(text))["kernel"].startswith("fused f32 tile=")


@pytest.mark.parametrize("seed", range(40))
def test_random_conv_plans(seed):
    from tests.random_programs import conv_case

    mod, host, dtypes, desc = conv_case(seed)
    assert xt.plan(mod)["kernel"].startswith("conv2d_nhwc")


@pytest.mark.parametrize("seed", range(40))
def test_random_gemm_plans_onto_the_gemm_kernel(seed):
    from tests.random_programs import gemm_case

    mod, host, dtypes, out, desc = gemm_case(seed)
    assert xt.plan(mod)["kernel"].startswith("gemm")


@pytest.mark.parametrize("seed", range(30))
def test_random_wide_cases_plan(seed):
    from tests.random_programs import wide_conv_case, wide_gemm_case

    mod, host, dtypes, desc = wide_conv_case(seed)
    assert xt.plan(mod)["kernel"].startswith("conv2d_nhwc")
    mod, host, dtypes, out, desc = wide_gemm_case(seed)
    assert xt.plan(mod)["kernel"].startswith("gemm")
