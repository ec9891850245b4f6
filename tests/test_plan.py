"""Launch planner: which kernel a tile program gets, and the host-side checks
that keep every kernel inside its buffers (runs without a GPU)."""

from __future__ import annotations

import pytest

import xtile_amd as xt
from xtile_amd import kernels as K


@pytest.mark.parametrize(
    "name,kernel,nbytes,nflops",
    [
        ("c1_add", "ew_binary op=add f32 tile=32x64 flat=1048576 grid=(32,16,1)", 12582912, 0),
        ("c2_softmax", "row_softmax f32 tile=1x4096 grid=(8192,1,1)", 268435456, 0),
        ("c3_matmul_f16", "gemm f16->f32 tile=128x128 k=4096 grid=(32,32,1)", 134217728, 137438953472),
        ("c4_conv2d_f16", "conv2d_nhwc f16->f32 tile=1x4x56x64 filter=3x3x64x64 grid=(32,14,1)", 38608896, 7398752256),
        ("c5_matmul_bf16", "gemm bf16->f32 tile=256x128 k=4096 grid=(86,16,1)", 304087040, 369367187456),
    ],
)
def test_benchmark_configs_plan(name, kernel, nbytes, nflops):
    """Algorithmic work per launch: C1 reads two and writes one 1024^2 f32
    array; C2 reads and writes 8192 x 4096 f32; C3 / C5 are 2 M N K FLOP; C4
    is 2 x pixels x Cout x (3 * 3 * 64) FLOP over input + filter + output
    bytes."""
    p = xt.plan(K.CONFIGS[name]())
    assert p["kernel"] == kernel
    assert p["bytes"] == nbytes
    assert p["flops"] == nflops


def test_reference_kernel_forms_plan():
    assert xt.plan(K.add_rows(128, 128, 64))["kernel"].startswith("ew_binary")
    assert xt.plan(K.softmax(128, 64, 64))["kernel"] == "row_softmax f32 tile=64x64 grid=(2,1,1)"


def _ew_program(rows, cols, th, tw, grid, swap_b=False, shared_b=0):
    """store(load A + load B) over rows x cols f32 memrefs, th x tw tiles;
    B's tile index optionally transposed or shared."""
    from xtile_amd import Array, bid, convert, float32, kernel, load, store

    @kernel
    def prog(a, b, c):
        x = bid(0)
        y = bid(1)
        ta = load(a, index=(x, y), shape=(th, tw))
        tb = load(b, index=(y, x) if swap_b else (x, y), shape=(th, tw), shared=shared_b)
        store(c, index=(x, y), tile=ta + tb)

    t = Array(shape=(rows, cols), dtype=float32)
    return convert(prog, args=(t, t, t), grid=(grid[0], grid[1], 1))


@pytest.mark.parametrize(
    "rows,cols,th,tw,grid,flat",
    [
        (1024, 1024, 32, 64, (32, 16), 1024 * 1024),  # C1: the tiles cover the whole array
        (64, 256, 64, 256, (1, 1), 64 * 256),          # one Block
        (256, 128, 8, 128, (32, 1), 256 * 128),        # full-width row tiles
        (128, 64, 16, 32, (4, 2), 64 * 64),            # the grid covers the first 64 full rows: one run
        (128, 64, 32, 16, (4, 2), 0),                  # the grid covers half of each row: holes
        (128, 64, 16, 16, (8, 4), 128 * 64),           # every tile, Blocks of 16 x 16
    ],
)
def test_elementwise_flat_run(rows, cols, th, tw, grid, flat):
    """The Blocks of store(load A + load B) run as one flat stream exactly when
    their tiles cover one contiguous run of every operand, each element once, at
    the same positions."""
    kernel = xt.plan(_ew_program(rows, cols, th, tw, grid))["kernel"]
    assert kernel.startswith("ew_binary")
    assert (f" flat={flat} " in kernel) if flat else ("flat=" not in kernel)


def test_elementwise_flat_run_needs_the_same_walk():
    """A transposed Block index in one operand or a shared operand whose index
    the leader rule pins: B's tiles no longer sit at A's and C's positions of
    the run, so the tiled kernel keeps the Blocks."""
    base = dict(rows=128, cols=128, th=32, tw=32, grid=(4, 4))
    assert " flat=16384 " in xt.plan(_ew_program(**base))["kernel"]
    assert "flat=" not in xt.plan(_ew_program(**base, swap_b=True))["kernel"]
    assert "flat=" not in xt.plan(_ew_program(**base, shared_b=1))["kernel"]
    # with one Block along axis 0 the shared rule changes nothing: B walks like A
    assert " flat=4096 " in xt.plan(_ew_program(32, 128, 32, 32, (1, 4), shared_b=1))["kernel"]


def test_compile_returns_module_and_keeps_text():
    m = K.softmax(16, 256, 1)
    before = str(m)
    assert xt.compile(m) is m
    assert str(m) == before


def test_out_of_bounds_tiles_are_rejected():
    # kernels/add.py with rows not a multiple of the 64-row tile: the last tile overruns
    with pytest.raises(NotImplementedError, match="exceeds extent"):
        xt.plan(K.add_rows(100, 128, 64))


def test_unsupported_program_names_its_ops():
    """Two convolutions in one Block: no kernel takes it, and the error lists the ops."""
    text = K.conv2d(1, 8, 8, 32, 32, 3, 3, 4, 8).__str__()
    lines = text.splitlines()
    conv = next(i for i, l in enumerate(lines) if "xt.load_conv2d" in l)
    second = lines[conv].replace("%load_conv =", "%load_conv2 =")
    m = xt.parse("\n".join(lines[: conv + 1] + [second] + lines[conv + 1 :]))
    with pytest.raises(NotImplementedError, match="unsupported tile program.*xt.load_conv2d xt.load_conv2d"):
        xt.plan(m)


def test_conv_inside_a_larger_program_gives_the_conv_form():
    text = K.conv2d(1, 8, 8, 32, 32, 3, 3, 4, 8).__str__()
    text = text.replace("xt.store(%load_conv,", "%e = xt.exp(%load_conv) : tensor<1x4x8x32xf32> -> tensor<1x4x8x32xf32>\n  xt.store(%e,")
    with pytest.raises(NotImplementedError, match=r"conv2d programs must be store\(load_conv2d"):
        xt.plan(xt.parse(text))


@pytest.mark.parametrize(
    "name,kernel,interp",
    [
        ("unary_and_shape", "staged f32 threads=256 lds=", "tile_vm f32 insts=12 loads=2 stores=3 lds="),
        ("column_reduce", "fused f32 tile=8x8 threads=8x2 vw=4 insts=3 ", "fused f32 tile=8x8 threads=8x2 vw=4 insts=3 "),
        ("divide_kernel", "fused f32 tile=8x8 threads=8x2 vw=4 insts=5 ", "fused f32 tile=8x8 threads=8x2 vw=4 insts=5 "),
        ("compute_ops", "staged f32 threads=256 lds=4352B mfma=i8 insts=5", "tile_vm f32 insts=5 loads=3 stores=1 lds="),
    ],
)
def test_general_programs_plan_onto_compiled_kernels(monkeypatch, name, kernel, interp):
    """Programs of loads, stores, unary / binary ops and reductions over one
    [R, C] tile and its broadcasts are compiled into a fused kernel; the rest
    (rank-3 tiles, matmul / mma, transposes) into a staged kernel, or run on
    the interpreter with XTILE_AMD_STAGE=0."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    k, args, grid, db = programs(dsl)[name]
    m = xt.convert(k, args=args, grid=grid, double_buffering=db)
    assert xt.plan(m)["kernel"].startswith(kernel)
    monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    m = xt.convert(k, args=args, grid=grid, double_buffering=db)
    assert xt.plan(m)["kernel"].startswith(interp)


def test_staged_plans():
    """The staged kernel's choices: f16 operands as loaded take the f16 MFMA,
    the f32 probabilities the f32 MFMA; algorithmic bytes count a head's
    shared K and V tiles once."""
    m = K.attention(512, 128, 128, 64, 64)
    p = xt.plan(m)
    assert p["kernel"].startswith("staged f32 threads=256 lds=") and "mfma=f32,f16" in p["kernel"]
    q = 512 * 128 * 64 * 2
    assert p["bytes"] == q + q + 2 * (512 * 128 * 64 * 4)  # Q, K (f16), V, O (f32): each tile once
    assert p["flops"] == 2 * (2 * 512 * 128 * 128 * 64)
    m = K.attention(2, 48, 33, 20, 16, qk=xt.float32)
    assert "mfma=f32 " in xt.plan(m)["kernel"]


def test_staged_row_segments(tmp_path, monkeypatch):
    """The staged generator computes the attention's softmax (row max,
    subtract, exp, row sum, reciprocal, scale) in registers as one step with
    four lanes a row, so the kernel has three barriers: after the loads,
    after Q K^T and after the softmax."""
    monkeypatch.setenv("XTILE_AMD_JIT_CACHE", str(tmp_path))
    xt.plan(K.attention(1000, 64, 64, 64, 64))  # a grid no other test plans: compiled here, written here
    (src,) = [f.read_text() for f in tmp_path.glob("*.hip")]
    assert "// rows 5-10: 4 lanes a row of [64,64], 16 elements a lane, in registers" in src
    body = src[src.index("xt_fused(FusedArgs a)"):]
    assert body.count("xbar();") == 3 and "__syncthreads" not in body


def test_interpreter_programs_and_lds_budget(monkeypatch):
    assert xt.plan(K.layernorm(128, 64, 64))["kernel"].startswith("fused f32 tile=64x64 threads=32x16 vw=4 insts=17")
    assert xt.plan(K.layernorm(8192, 4096, 1))["kernel"].startswith("fused f32 tile=1x4096 threads=1x512 vw=4")
    # fused kernels hold values in registers, so the interpreter's LDS budget does not bind them
    assert xt.plan(K.layernorm(8192, 4096, 4))["kernel"].startswith("fused f32 tile=4x4096 threads=1x512 vw=4")
    assert xt.plan(K.column_softmax(64, 128, 32))["kernel"].startswith("fused f32 tile=64x32 threads=64x8")
    assert xt.plan(K.bias_add(128, 256))["kernel"].startswith("fused f32 tile=32x64 threads=32x16")
    monkeypatch.setenv("XTILE_AMD_FUSE", "0")
    assert xt.plan(K.layernorm(128, 64, 64))["kernel"].startswith(
        "tile_vm f32 insts=17 loads=5 stores=1 lds=50208B (not fused: XTILE_AMD_FUSE=0)")
    with pytest.raises(NotImplementedError, match="KB of LDS"):
        xt.plan(K.layernorm(8192, 4096, 4))
    monkeypatch.delenv("XTILE_AMD_FUSE")
    # live tiles beyond 160 KB of LDS are refused on the host
    with pytest.raises(NotImplementedError, match="KB of LDS"):
        xt.plan(K.layernorm(512, 256, 256))


def test_epilogue_matmul_plans():
    """The reference's own matmul program (traced by the reference DSL):
    i8 x i8 -> * scale + bias -> astype(int8) maps onto the epilogue GEMM."""
    from tests.golden.dsl_programs import programs
    from xtile_amd import dsl

    kernel, args, grid, db = programs(dsl)["matmul_int8_epilogue"]
    m = xt.convert(kernel, args=args, grid=grid, double_buffering=db)
    assert xt.plan(m)["kernel"] == "gemm i8->f32 tile=64x64 k=256 epilogue=scale,bias,ftoi->i8 grid=(16,8,1)"


_MM_EXP = """
func.func @k(%a: memref<MxKxf16>, %b: memref<KxNxf16>, %c: memref<MxNxf32>) attributes {xt.grid = array<i32: 1, 1, 1>} {
  %z = arith.constant 0 : i32
  %0 = xt.load(%a, %z, %z) : (memref<MxKxf16>, i32, i32) -> tensor<MxKxf16>
  %1 = xt.load(%b, %z, %z) : (memref<KxNxf16>, i32, i32) -> tensor<KxNxf16>
  %2 = xt.matmul(%0, %1) : tensor<MxKxf16>, tensor<KxNxf16> -> tensor<MxNxf32>
  %3 = xt.exp(%2) : tensor<MxNxf32> -> tensor<MxNxf32>
  xt.store(%3, %c, %z, %z) : (tensor<MxNxf32>, memref<MxNxf32>, i32, i32) -> ()
  func.return
}"""


def _mm_exp(m, k, n):
    return xt.parse(_MM_EXP.replace("MxK", f"{m}x{k}").replace("KxN", f"{k}x{n}").replace("MxN", f"{m}x{n}"))


def test_matmul_outside_the_gemm_forms_runs_compiled(monkeypatch):
    """A matmul followed by another op: the staged kernel (f16 MFMA on the
    operands as loaded), or the interpreter with XTILE_AMD_STAGE=0."""
    assert xt.plan(_mm_exp(64, 64, 64))["kernel"].startswith("staged f32 threads=256 lds=34816B mfma=f16 insts=5")
    monkeypatch.setenv("XTILE_AMD_STAGE", "0")
    assert xt.plan(_mm_exp(64, 64, 64))["kernel"].startswith("tile_vm f32 insts=5 loads=2 stores=1")


def test_unsupported_matmul_epilogue_is_reported():
    """Too large for the interpreter's LDS: both reasons are given."""
    with pytest.raises(NotImplementedError, match=r"matmul programs must be store\(\[ftoi\].*declines it too: "
                       r"tile program needs 320 KB of LDS"):
        xt.plan(_mm_exp(128, 256, 128))


def test_nova_stages_raise():
    m = xt.xt_to_nova(K.add(64, 64, 32, 32))
    with pytest.raises(NotImplementedError, match="x1 NPU lowering"):
        xt.nova_optimize(m)


def test_xt_to_nova_returns_the_same_module():
    """test/python/to_nova.py: the wrapper is returned, its text lowered."""
    m = xt.parse(
        """
        module {
          func.func @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {
            %0 = xt.add(%arg0, %arg0) : tensor<4xf32>, tensor<4xf32> -> tensor<4xf32>
            func.return %0 : tensor<4xf32>
          }
        }
        """
    )
    assert xt.xt_to_nova(m) is m
    assert "nova.elementwise 1 %arg0, %arg0" in str(m)


def test_save_compile_results(tmp_path, capsys):
    m = K.add(64, 128, 32, 64)
    xt.save_compile_results(m, str(tmp_path / "add"))
    files = sorted(p.name for p in (tmp_path / "add").iterdir())
    assert files == ["0_xt.mlir", "1_hip_plan.txt", "2_xt_serialize.mlir", "3_xt_to_nova.mlir"]
    assert "nova.elementwise" in (tmp_path / "add" / "3_xt_to_nova.mlir").read_text()
    assert "ew_binary" in (tmp_path / "add" / "1_hip_plan.txt").read_text()
    assert "compiled kernel ->" in capsys.readouterr().out


def test_shared_load_of_moving_tile_plans():
    """shared=1 with an index that moves along axis 0: the group leader's tile is used."""
    text = """
func.func @s(%a: memref<64x64xf32>, %b: memref<64x64xf32>, %c: memref<64x64xf32>) attributes {xt.grid = array<i32: 2, 2, 1>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%a, %bid#0, %bid#1) {shared = 1 : i64} : (memref<64x64xf32>, i32, i32) -> tensor<32x32xf32>
  %1 = xt.load(%b, %bid#0, %bid#1) : (memref<64x64xf32>, i32, i32) -> tensor<32x32xf32>
  %2 = xt.add(%0, %1) : tensor<32x32xf32>, tensor<32x32xf32> -> tensor<32x32xf32>
  xt.store(%2, %c, %bid#0, %bid#1) : (tensor<32x32xf32>, memref<64x64xf32>, i32, i32) -> ()
  func.return
}"""
    assert xt.plan(xt.parse(text))["kernel"].startswith("ew_binary")


@pytest.mark.parametrize(
    "prog,args,layout",
    [
        # 1899 float2 a row: no power-of-two thread row divides it, so 512 threads take
        # four vectors each and the last 149 of the fourth round are absent
        ("layernorm", (64, 3798, 1), "fused f32 tile=1x3798 threads=1x512 vw=2 ragged insts=17"),
        ("layernorm", (64, 1000, 1), "fused f32 tile=1x1000 threads=1x128 vw=4 ragged insts=17"),
        ("layernorm", (32, 130, 4), "fused f32 tile=4x130 threads=4x64 vw=2 ragged insts=17"),
        ("softmax", (64, 3798, 1), "fused f32 tile=1x3798 threads=1x512 vw=2 ragged insts=8"),
        # rows that a power-of-two thread row divides keep the exact layout
        ("layernorm", (8192, 4096, 1), "fused f32 tile=1x4096 threads=1x512 vw=4 workgroups=512 insts=17"),
        ("layernorm", (96, 48, 16), "fused f32 tile=16x48 threads=16x4 vw=4 insts=17"),
    ],
)
def test_fused_ragged_rows(prog, args, layout):
    """Rows whose vector count has no power-of-two divisor wide enough to keep a
    thread's share at 64 elements or fewer run on a ragged fused layout instead
    of the interpreter."""
    m = getattr(K, prog)(*args)
    assert xt.plan(m)["kernel"].startswith(layout)


def test_fused_kernels_are_compiled_into_the_code_object_cache(tmp_path, monkeypatch):
    """Planning a fused program compiles it with hiprtc (no GPU needed) and
    writes the code object and its source under XTILE_AMD_JIT_CACHE."""
    monkeypatch.setenv("XTILE_AMD_JIT_CACHE", str(tmp_path))
    # a shape no other test plans, so the in-process cache does not hold it
    assert xt.plan(K.layernorm(24, 40, 8))["kernel"].startswith("fused f32 tile=8x40 threads=8x2 vw=4")
    cos = list(tmp_path.glob("*.co"))
    srcs = list(tmp_path.glob("*.hip"))
    assert len(cos) == 1 and len(srcs) == 1 and cos[0].stem == srcs[0].stem
    assert cos[0].read_bytes()[:4] == b"\x7fELF"  # an AMDGPU code object
    assert 'extern "C" __global__' in srcs[0].read_text() and "xt_fused" in srcs[0].read_text()
    monkeypatch.setenv("XTILE_AMD_JIT_CACHE", "off")
    other = tmp_path / "none"
    xt.plan(K.layernorm(24, 80, 8))
    assert not other.exists() and len(list(tmp_path.glob("*.co"))) == 1


def test_softmax_rows_above_2048_need_float4_vectors():
    assert xt.plan(K.softmax(64, 4096, 1))["kernel"].startswith("row_softmax")
    assert xt.plan(K.softmax(64, 2047, 1))["kernel"].startswith("row_softmax")
    # 1899 float2 a row: the fused kernel's ragged layout (the interpreter before it)
    assert xt.plan(K.softmax(122, 3798, 2))["kernel"].startswith("fused f32 tile=2x3798 threads=1x512 vw=2 ragged")


def test_native_binding_has_the_reference_stage_names():
    """A reference facade pointed at this binding (xtile/__init__.py:130-168
    calls _native.nova_optimize ... nova_to_x1) gets NotImplementedError for
    a module and TypeError for anything else, never AttributeError."""
    from xtile_amd import _xtile as native

    m = K.add(64, 128, 32, 64)
    for name in ("nova_optimize", "nova_threading", "nova_barrier", "nova_allocate", "nova_to_x1"):
        stage = getattr(native, name)
        with pytest.raises(NotImplementedError, match="x1 NPU lowering"):
            stage(m)
        with pytest.raises(TypeError):
            stage("not a module")
        with pytest.raises(NotImplementedError):
            getattr(xt, name)(m)


def _add_program(rows, cols, th, tw, grid):
    return xt.parse(f"""
func.func @k(%a: memref<{rows}x{cols}xf32>, %b: memref<{rows}x{cols}xf32>, %c: memref<{rows}x{cols}xf32>) attributes {{xt.grid = array<i32: {grid[0]}, {grid[1]}, 1>}} {{
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%a, %bid#0, %bid#1) : (memref<{rows}x{cols}xf32>, i32, i32) -> tensor<{th}x{tw}xf32>
  %1 = xt.load(%b, %bid#0, %bid#1) : (memref<{rows}x{cols}xf32>, i32, i32) -> tensor<{th}x{tw}xf32>
  %2 = xt.add(%0, %1) : tensor<{th}x{tw}xf32>, tensor<{th}x{tw}xf32> -> tensor<{th}x{tw}xf32>
  xt.store(%2, %c, %bid#0, %bid#1) : (tensor<{th}x{tw}xf32>, memref<{rows}x{cols}xf32>, i32, i32) -> ()
  func.return
}}""")


def test_grid_beyond_one_launch_is_refused_before_any_device_call():
    """2^31 Blocks of 1x1 tiles over an 8 GiB array: the Block count is
    computed in 64 bits and the launcher refuses it (XT_ERR_ARGUMENT ->
    ValueError) before it makes any HIP call, so this runs without a GPU."""
    from xtile_amd import _xtile as native

    m = _add_program(65536, 32768, 1, 1, (65536, 32768))
    assert xt.plan(m)["kernel"].startswith("ew_binary")
    nbytes = 65536 * 32768 * 4
    fake = [0x10000, 0x20000, 0x30000]  # never dereferenced: the launch is refused first
    with pytest.raises(ValueError, match="exceeds one launch"):
        native.launch(m, None, fake, [nbytes] * 3)
    # just inside the limit (2^24 workgroups of 256 work-items) the plan is unchanged
    ok = _add_program(4096, 4096, 1, 1, (4096, 4095))
    assert xt.plan(ok)["kernel"].startswith("ew_binary")


INDEPENDENCE = """
func.func @k(%a: memref<64x64xf32>, %c: memref<64x64xf32>) attributes {{xt.grid = array<i32: 2, 2, 1>}} {{
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %c0 = arith.constant 0 : i32
  %0 = xt.load(%a, {load}) : (memref<64x64xf32>, i32, i32) -> tensor<32x32xf32>
  %1 = xt.exp(%0) : tensor<32x32xf32> -> tensor<32x32xf32>
  xt.store(%1, %c, {store}) : (tensor<32x32xf32>, memref<64x64xf32>, i32, i32) -> ()
  func.return
}}"""


def test_blocks_storing_different_values_to_one_tile_are_refused():
    """Every Block stores to tile (0, bid1) a value that depends on bid0: the
    reference's serial order keeps the last Block's (XTSerialize.cpp:68-104),
    concurrent Blocks race, so the plan is refused."""
    m = xt.parse(INDEPENDENCE.format(load="%bid#0, %bid#1", store="%c0, %bid#1"))
    with pytest.raises(NotImplementedError, match="grid axis 0 store different values"):
        xt.plan(m)
    # the same store of a value that does not depend on bid0 writes equal values: allowed
    same = xt.parse(INDEPENDENCE.format(load="%c0, %bid#1", store="%c0, %bid#1"))
    assert xt.plan(same)["kernel"]
    # a shared=1 load reads the leader's tile, so its value does not vary along axis 0
    shared = xt.parse(INDEPENDENCE.format(load="%bid#0, %bid#1", store="%c0, %bid#1").replace(
        "%0 = xt.load(%a, %bid#0, %bid#1)", "%0 = xt.load(%a, %bid#0, %bid#1) {shared = 1 : i64}"))
    assert xt.plan(shared)["kernel"]


def test_in_place_programs_must_touch_only_their_own_tile():
    """A memref loaded and stored: allowed at the same tile (in place), refused
    when Blocks read tiles other Blocks store (a transposed in-place store)."""
    inplace = INDEPENDENCE.format(load="%bid#0, %bid#1", store="%bid#0, %bid#1").replace("%c,", "%a,")
    assert xt.plan(xt.parse(inplace))["kernel"]
    transposed = INDEPENDENCE.format(load="%bid#0, %bid#1", store="%bid#1, %bid#0").replace("%c,", "%a,")
    with pytest.raises(NotImplementedError, match="stored and also accessed at another tile"):
        xt.plan(xt.parse(transposed))
