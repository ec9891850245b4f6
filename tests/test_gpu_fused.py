"""GPU parity of fused tile programs (csrc/fused.cpp, compiled by hiprtc).

Programs of loads, stores, unary / binary ops and reductions over one [R, C]
tile and its [1, C] / [R, 1] / [1, 1] broadcasts are compiled into one kernel
that keeps values in registers.  These tests cover the layouts the generator
picks: a row spread over four or eight waves (cross-wave row reduction
through LDS),
several rows per thread, a column reduction over 64 or 256 threads of a
column,
[R, 1] and [1, 1] stores, ragged rows (a vector count no power-of-two thread
row divides: the last vectors of a thread row absent), a buffer not aligned to
the row vectors (which runs the program's scalar-access variant instead), and
agreement with the interpreter (XTILE_AMD_FUSE=0).

Bars: layernorm within 2e-5 absolute of the oracle (inputs of unit scale, a
different summation order); column softmax within 1e-5 relative; programs
without reductions bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

import xtile_amd as xt
from tests.conftest import oracle_threads
from tests.gpu_util import run_gpu, run_oracle
from xtile_amd import kernels as K

pytestmark = pytest.mark.gpu


def _ln_inputs(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1.5, (rows, cols)).astype(np.float32)
    g = rng.normal(1, 0.2, (1, cols)).astype(np.float32)
    b = rng.normal(0, 0.2, (1, cols)).astype(np.float32)
    return [x, g, b, np.full((1, 1), 1.0 / cols, np.float32), np.full((1, 1), 1e-5, np.float32), np.zeros_like(x)]


@pytest.mark.parametrize(
    "rows,cols,trow,layout",
    [
        (256, 4096, 1, "tile=1x4096 threads=1x512"),   # a row over 8 waves
        (256, 4096, 4, "tile=4x4096 threads=1x512"),   # 4 rows per thread, 32 values each
        (512, 1024, 2, "tile=2x1024 threads=2x256"),   # two rows, each over 4 waves
        (96, 48, 16, "tile=16x48 threads=16x4"),       # 48 columns: 12 vectors, 4 threads a row
        # more Blocks than the chip holds: 2048 workgroups walk 8192 Blocks with gamma / beta in registers
        (8192, 1024, 1, "tile=1x1024 threads=1x256 vw=4 workgroups=2048"),
        # 512 workgroups walk 5000 Blocks: the last pass leaves most workgroups without a Block
        (5000, 4096, 1, "tile=1x4096 threads=1x512 vw=4 workgroups=512"),
    ],
)
def test_fused_layernorm(cuda, rows, cols, trow, layout):
    m = K.layernorm(rows, cols, trow)
    assert xt.plan(m)["kernel"].startswith("fused f32 " + layout)
    bufs = _ln_inputs(rows, cols, 41)
    got = run_gpu(m, bufs, ["f32"] * 6, cuda, case=f"fused layernorm {rows}x{cols}/{trow}")[5]
    want = run_oracle(m, bufs, oracle_threads())[5]
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("rows,cols,tcol", [(512, 64, 32), (256, 256, 8)])
def test_fused_column_softmax(cuda, rows, cols, tcol):
    m = K.column_softmax(rows, cols, tcol)
    desc = xt.plan(m)["kernel"]
    assert desc.startswith("fused"), desc
    rng = np.random.default_rng(42)
    x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
    got = run_gpu(m, [x, np.zeros_like(x)], ["f32"] * 2, cuda, case=f"fused column softmax {rows}x{cols}/{tcol}")[1]
    want = run_oracle(m, [x, np.zeros_like(x)], oracle_threads())[1]
    assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
    np.testing.assert_allclose(got.sum(axis=0), 1.0, atol=1e-5)


_STATS = """
func.func @stats(%x: memref<64x256xf32>, %rs: memref<64x1xf32>, %cm: memref<4x256xf32>, %t: memref<4x1xf32>, %y: memref<64x256xi8>) attributes {xt.grid = array<i32: 4, 1, 1>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %z = arith.constant 0 : i32
  %0 = xt.load(%x, %bid#0, %z) : (memref<64x256xf32>, i32, i32) -> tensor<16x256xf32>
  %1 = xt.reduce_sum(%0) {axis = 1 : i64} : tensor<16x256xf32> -> tensor<16x1xf32>
  xt.store(%1, %rs, %bid#0, %z) : (tensor<16x1xf32>, memref<64x1xf32>, i32, i32) -> ()
  %2 = xt.reduce_max(%0) {axis = 0 : i64} : tensor<16x256xf32> -> tensor<1x256xf32>
  xt.store(%2, %cm, %bid#0, %z) : (tensor<1x256xf32>, memref<4x256xf32>, i32, i32) -> ()
  %3 = xt.reduce_max(%1) {axis = 0 : i64} : tensor<16x1xf32> -> tensor<1x1xf32>
  xt.store(%3, %t, %bid#0, %z) : (tensor<1x1xf32>, memref<4x1xf32>, i32, i32) -> ()
  %4 = xt.sub(%0, %1) : tensor<16x256xf32>, tensor<16x1xf32> -> tensor<16x256xf32>
  %5 = xt.ftoi(%4) : tensor<16x256xf32> -> tensor<16x256xi8>
  xt.store(%5, %y, %bid#0, %z) : (tensor<16x256xi8>, memref<64x256xi8>, i32, i32) -> ()
  func.return
}
"""


def test_fused_row_column_and_scalar_stores(cuda):
    """Row sums ([R, 1] store by one thread a row), column maxima of each Block ([1, C]
    store), the largest row sum ([1, 1] store by one thread) and an i8 store
    (ftoi: round, saturate) of a two-sided broadcast difference."""
    m = xt.parse(_STATS)
    desc = xt.plan(m)["kernel"]
    assert desc.startswith("fused"), desc
    rng = np.random.default_rng(43)
    x = rng.normal(0, 1, (64, 256)).astype(np.float32)
    bufs = [x, np.zeros((64, 1), np.float32), np.zeros((4, 256), np.float32), np.zeros((4, 1), np.float32),
            np.zeros((64, 256), np.int8)]
    dts = ["f32", "f32", "f32", "f32", "i8"]
    got = run_gpu(m, bufs, dts, cuda, case="fused stats")
    want = run_oracle(m, bufs, 1)
    scale = np.abs(x).sum(axis=1).max()
    np.testing.assert_allclose(got[1], want[1], rtol=0, atol=1e-5 * scale)
    assert np.array_equal(got[2], want[2])  # max is exact in any order
    np.testing.assert_allclose(got[3], want[3], rtol=0, atol=1e-5 * scale)
    # i8 of x - rowsum: one rounding of a difference whose rowsum may differ in the last bits
    d = np.abs(got[4].astype(np.int32) - want[4].astype(np.int32))
    assert d.max() <= 1


_STATS100 = _STATS.replace("x256x", "x100x").replace("x256x", "x100x").replace("256x", "100x")


def test_fused_ragged_row_column_and_scalar_stores(cuda):
    """The stats program over 100 columns (25 float4 a row): a ragged layout of
    16 threads a row, two vectors each, the second present for 9 of the 16.
    Absent vectors are neither stored ([R, C] i8 and [1, C] stores) nor part of
    the row sums; the column maxima of present columns are exact."""
    m = xt.parse(_STATS100)
    desc = xt.plan(m)["kernel"]
    assert desc.startswith("fused f32 tile=16x100 threads=16x16 vw=4 ragged"), desc
    rng = np.random.default_rng(44)
    x = rng.normal(0, 1, (64, 100)).astype(np.float32)
    # sentinels: a store to an absent column would overwrite them
    bufs = [x, np.zeros((64, 1), np.float32), np.full((4, 100), 7.0, np.float32), np.zeros((4, 1), np.float32),
            np.full((64, 100), 5, np.int8)]
    dts = ["f32", "f32", "f32", "f32", "i8"]
    got = run_gpu(m, bufs, dts, cuda, case="fused stats ragged 64x100")
    want = run_oracle(m, bufs, 1)
    scale = np.abs(x).sum(axis=1).max()
    np.testing.assert_allclose(got[1], want[1], rtol=0, atol=1e-5 * scale)
    assert np.array_equal(got[2], want[2])
    np.testing.assert_allclose(got[3], want[3], rtol=0, atol=1e-5 * scale)
    d = np.abs(got[4].astype(np.int32) - want[4].astype(np.int32))
    assert d.max() <= 1


@pytest.mark.parametrize(
    "rows,cols,trow,layout",
    [
        (64, 3798, 1, "tile=1x3798 threads=1x512 vw=2 ragged"),  # 1899 float2: 4 rounds of 512, the last 363 present
        (64, 1000, 1, "tile=1x1000 threads=1x128 vw=4 ragged"),   # 250 float4 over 128 threads
        (32, 130, 4, "tile=4x130 threads=4x64 vw=2 ragged"),      # 65 float2: one present in the second round
        (64, 4100, 1, "tile=1x4100 threads=1x512 vw=4 ragged"),   # 1025 float4: one vector in the third round
        (8192, 2050, 1, "tile=1x2050 threads=1x512 vw=2 ragged workgroups="),  # Block walk, gamma / beta ragged
    ],
)
def test_fused_ragged_layernorm(cuda, monkeypatch, rows, cols, trow, layout):
    """Layernorm over rows whose vector count no power-of-two thread row
    divides: against the oracle, and against the interpreter (XTILE_AMD_FUSE=0)."""
    m = K.layernorm(rows, cols, trow)
    assert xt.plan(m)["kernel"].startswith("fused f32 " + layout)
    bufs = _ln_inputs(rows, cols, 45)
    got = run_gpu(m, bufs, ["f32"] * 6, cuda, case=f"fused ragged layernorm {rows}x{cols}/{trow}")[5]
    want = run_oracle(m, bufs, oracle_threads())[5]
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    if rows <= 64:
        monkeypatch.setenv("XTILE_AMD_FUSE", "0")
        m2 = K.layernorm(rows, cols, trow)
        assert xt.plan(m2)["kernel"].startswith("tile_vm")
        vm = run_gpu(m2, bufs, ["f32"] * 6, cuda, case=f"interpreted layernorm {rows}x{cols}/{trow}")[5]
        np.testing.assert_allclose(got, vm, rtol=0, atol=2e-5)


@pytest.mark.parametrize("rows,cols", [(64, 3798), (256, 2050)])
def test_fused_ragged_softmax(cuda, rows, cols):
    """Row softmax over rows of an odd number of float2 vectors (the float4
    softmax kernel declines them)."""
    m = K.softmax(rows, cols, 1)
    assert xt.plan(m)["kernel"].startswith("fused f32 tile=1x%d threads=1x512 vw=2 ragged" % cols)
    rng = np.random.default_rng(46)
    x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
    got = run_gpu(m, [x, np.zeros_like(x)], ["f32"] * 2, cuda, case=f"fused ragged softmax {rows}x{cols}")[1]
    want = run_oracle(m, [x, np.zeros_like(x)], oracle_threads())[1]
    assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
    np.testing.assert_allclose(got.sum(axis=1), 1.0, atol=1e-5)


_CENTER = """
func.func @center(%x: memref<8192x4096xf32>, %b: memref<1x4096xf32>, %y: memref<8192x4096xf32>) attributes {xt.grid = array<i32: 8192, 1, 1>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %z = arith.constant 0 : i32
  %0 = xt.load(%x, %bid#0, %z) : (memref<8192x4096xf32>, i32, i32) -> tensor<1x4096xf32>
  %1 = xt.load(%b, %z, %z) {shared = 1 : i64} : (memref<1x4096xf32>, i32, i32) -> tensor<1x4096xf32>
  %2 = xt.reduce_max(%0) {axis = 1 : i64} : tensor<1x4096xf32> -> tensor<1x1xf32>
  %3 = xt.sub(%0, %2) : tensor<1x4096xf32>, tensor<1x1xf32> -> tensor<1x4096xf32>
  %4 = xt.add(%3, %1) : tensor<1x4096xf32>, tensor<1x4096xf32> -> tensor<1x4096xf32>
  xt.store(%4, %y, %bid#0, %z) : (tensor<1x4096xf32>, memref<8192x4096xf32>, i32, i32) -> ()
  func.return
}
"""


def test_fused_block_loop_with_one_lds_reduction_is_bit_exact(cuda):
    """x - rowmax(x) + b over 8192 rows: 512 workgroups walk the Blocks with
    b in registers, and the one LDS reduction region is reused Block after
    Block (a barrier closes each Block).  max, sub and add are exact in any
    order, so the result is bit-exact."""
    m = xt.parse(_CENTER)
    assert xt.plan(m)["kernel"].startswith("fused f32 tile=1x4096 threads=1x512 vw=4 workgroups=512")
    rng = np.random.default_rng(47)
    x = rng.normal(0, 1, (8192, 4096)).astype(np.float32)
    b = rng.normal(0, 1, (1, 4096)).astype(np.float32)
    got = run_gpu(m, [x, b, np.zeros_like(x)], ["f32"] * 3, cuda, case="fused center 8192x4096")[2]
    want = (x - x.max(axis=1, keepdims=True)) + b
    assert np.array_equal(got, want)


def test_fused_matches_the_interpreter_bit_exact_without_reductions(cuda, monkeypatch):
    rng = np.random.default_rng(44)
    a = rng.normal(0, 1, (128, 256)).astype(np.float32)
    v = rng.normal(0, 1, (1, 256)).astype(np.float32)
    fused = K.bias_add(128, 256)
    assert xt.plan(fused)["kernel"].startswith("fused")
    got = run_gpu(fused, [a, v, np.zeros_like(a)], ["f32"] * 3, cuda, case="fused bias add")[2]
    monkeypatch.setenv("XTILE_AMD_FUSE", "0")
    interp = K.bias_add(128, 256)
    assert xt.plan(interp)["kernel"].startswith("tile_vm")
    ref = run_gpu(interp, [a, v, np.zeros_like(a)], ["f32"] * 3, cuda, case="interpreted bias add")[2]
    assert np.array_equal(got, ref)
    assert np.array_equal(got, a + v)


def test_fused_and_interpreted_layernorm_agree(cuda, monkeypatch):
    bufs = _ln_inputs(128, 64, 45)
    got = run_gpu(K.layernorm(128, 64, 64), bufs, ["f32"] * 6, cuda, case="fused layernorm 128x64")[5]
    monkeypatch.setenv("XTILE_AMD_FUSE", "0")
    ref = run_gpu(K.layernorm(128, 64, 64), bufs, ["f32"] * 6, cuda, case="interpreted layernorm 128x64")[5]
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-5)


def test_misaligned_buffer_runs_the_scalar_variant(cuda):
    """A buffer offset by one f32 cannot be read as 16-byte vectors: the
    launch takes the program's scalar-access variant (vw = 1, built on first
    use) and the result is unchanged."""
    import torch

    m = K.bias_add(128, 256)
    assert "vw=4" in xt.plan(m)["kernel"]
    rng = np.random.default_rng(46)
    a = rng.normal(0, 1, (128, 256)).astype(np.float32)
    v = rng.normal(0, 1, (1, 256)).astype(np.float32)
    print("[gpu] misaligned bias add", flush=True)
    store = torch.zeros(128 * 256 + 1, dtype=torch.float32, device=cuda)
    out = store[1:].view(128, 256)
    assert out.data_ptr() % 16 == 4
    xt.launch(m, torch.from_numpy(a).to(cuda), torch.from_numpy(v).to(cuda), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), a + v)


def test_misaligned_buffer_of_a_program_the_interpreter_declines(cuda):
    """Layernorm over 4 x 4096 Blocks needs more LDS than the interpreter has,
    so before the scalar variant a misaligned buffer made the launch fail;
    now it runs with scalar row accesses and matches the oracle."""
    import torch

    m = K.layernorm(256, 4096, 4)
    desc = xt.plan(m)["kernel"]
    assert desc.startswith("fused f32 tile=4x4096 threads=1x512 vw=4"), desc
    bufs = _ln_inputs(256, 4096, 48)
    want = run_oracle(m, bufs, oracle_threads())[5]
    print("[gpu] misaligned layernorm 256x4096/4", flush=True)
    store = torch.zeros(256 * 4096 + 1, dtype=torch.float32, device=cuda)
    x = store[1:].view(256, 4096)
    assert x.data_ptr() % 16 == 4
    x.copy_(torch.from_numpy(bufs[0]).to(cuda))
    dev = [x] + [torch.from_numpy(b).to(cuda) for b in bufs[1:]]
    xt.launch(m, *dev)
    torch.cuda.synchronize()
    np.testing.assert_allclose(dev[5].cpu().numpy(), want, rtol=0, atol=2e-5)


def test_misaligned_softmax_rows_above_2048_run_on_the_interpreter(cuda):
    """Rows of 4096 floats are planned onto the float4 softmax kernel; a view
    with a 4-byte storage offset cannot be read as float4, so that launch
    runs on the interpreter lowering the plan keeps beside it (before, the
    launch was refused as 'row too long')."""
    import torch

    m = K.softmax(64, 4096, 1)
    assert xt.plan(m)["kernel"].startswith("row_softmax")
    rng = np.random.default_rng(47)
    x = rng.normal(0, 2, (64, 4096)).astype(np.float32)
    print("[gpu] misaligned softmax 64x4096", flush=True)
    store = torch.zeros(64 * 4096 + 1, dtype=torch.float32, device=cuda)
    inp = store[1:].view(64, 4096)
    assert inp.data_ptr() % 16 == 4
    inp.copy_(torch.from_numpy(x).to(cuda))
    out = torch.zeros(64, 4096, dtype=torch.float32, device=cuda)
    xt.launch(m, inp, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = run_oracle(m, [x, np.zeros_like(x)], 4)[1]
    assert np.max(np.abs(got - want) / np.abs(want)) <= 1e-5
