"""Native xt IR: parser, printer, verifier, passes, xt-opt and the C ABI.

Verifier diagnostics restate lib/xt/XTOps.cpp / XTDialect.cpp word for word;
serialize follows lib/xt/XTSerialize.cpp; canonicalize lib/xt/XTOps.cpp:399-449.
When the reference tree is mounted (build container only) its own lit files
test/xt/*.mlir are run through xt-opt + FileCheck as well.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import xtile_amd as xt
from xtile_amd import _xtile

ROOT = Path(__file__).resolve().parents[1]
XT_OPT = ROOT / "xtile_amd" / "lib" / "xt-opt"
FILECHECK = shutil.which("FileCheck") or "/opt/rocm/lib/llvm/bin/FileCheck"
REF_TESTS = Path("/root/reference/test/xt")


def xt_opt(args, text):
    p = subprocess.run([str(XT_OPT), *args, "-"], input=text, capture_output=True, text=True, timeout=60)
    return p.returncode, p.stdout, p.stderr


SERIAL = """
func.func @g(%src: memref<128x16xf32>, %dst: memref<128x16xf32>) attributes {xt.grid = array<i32: 2, 2, 1>} {
  %bid:3 = xt.get_tile_block_id : i32, i32, i32
  %0 = xt.load(%src, %bid#0, %bid#1) SHARED : (memref<128x16xf32>, i32, i32) -> tensor<16x16xf32>
  xt.store(%0, %dst, %bid#0, %bid#1) : (tensor<16x16xf32>, memref<128x16xf32>, i32, i32) -> ()
  func.return
}
"""


# -- parse / print ---------------------------------------------------------------


def test_round_trip_is_stable():
    src = SERIAL.replace("SHARED", "{shared = 1 : i64}")
    m = xt.parse(src)
    a = xt._module_asm(m)
    b = xt._module_asm(xt.parse(a))
    assert a == b
    assert "{shared = 1 : i64}" in a
    assert "xt.grid = array<i32: 2, 2, 1>" in a


def test_parse_error_is_value_error():
    with pytest.raises(ValueError, match="failed to parse test module"):
        xt.parse("func.func @f( {")
    with pytest.raises(ValueError, match="custom op 'xt.free' is unknown"):
        xt.parse("func.func @f(%a: tensor<4xf32>) {\n  xt.free(%a) : tensor<4xf32>\n  func.return\n}")


def test_wrong_object_is_type_error():
    with pytest.raises(TypeError):
        _xtile._module_asm(object())
    with pytest.raises(TypeError):
        _xtile.xt_serialize("module {}")


@pytest.mark.parametrize(
    "body,msg",
    [
        ("%0 = xt.load(%a, %z, %z) : (memref<64x16xf32>, i32, i32) -> tensor<16xf32>",
         "'xt.load' op coordinate count must match tensor rank"),
        ("%0 = xt.load(%a, %z, %z) : (memref<64x16xf32>, i32, i32) -> tensor<16x16xi8>",
         "requires matching memref/tensor element types"),
        ("%0 = xt.load(%a, %z, %z) {shared = 3 : i64} : (memref<64x16xf32>, i32, i32) -> tensor<16x16xf32>",
         "shared attribute must be 0, 1, or 2"),
        ("%0 = xt.load(%a, %z, %z) : (memref<64x16xf32>, i32, i32) -> tensor<16x16xf32>\n"
         "  %1 = xt.exp(%0) : tensor<16x16xf32> -> tensor<16x8xf32>",
         "requires operand and result tensor types to match"),
        ("%0 = xt.load(%a, %z, %z) : (memref<64x16xf32>, i32, i32) -> tensor<16x16xf32>\n"
         "  %1 = xt.reduce_max(%0) {axis = 1 : i64} : tensor<16x16xf32> -> tensor<16x16xf32>",
         "reduce result shape must match input shape except for the reduced dimension, which must be 1"),
        ("%0 = xt.load(%a, %z, %z) : (memref<64x16xf32>, i32, i32) -> tensor<16x16xf32>\n"
         "  %1 = xt.matmul(%0, %0) : tensor<16x16xf32>, tensor<16x16xf32> -> tensor<16x8xf32>",
         "result shape must match matmul output shape"),
    ],
)
def test_verifier_messages(body, msg):
    text = (
        "func.func @f(%a: memref<64x16xf32>) {\n  %z = arith.constant 0 : i32\n  " + body + "\n  func.return\n}"
    )
    with pytest.raises(ValueError) as ei:
        xt.parse(text)
    assert msg in str(ei.value)


def test_grid_attribute_rules():
    with pytest.raises(ValueError, match="xt.grid must have exactly 3 entries"):
        xt.parse("func.func @f() attributes {xt.grid = array<i32: 1, 2>} {\n  func.return\n}")
    with pytest.raises(ValueError, match="xt.grid entries must be positive"):
        xt.parse("func.func @f() attributes {xt.grid = array<i32: 1, 0, 1>} {\n  func.return\n}")
    with pytest.raises(ValueError, match="only valid on func.func"):
        xt.parse("module attributes {xt.grid = array<i32: 1, 1, 1>} {\n}")


def test_narrow_float_matmul_extension_verifies():
    text = (
        "func.func @f(%a: tensor<16x32xbf16>, %b: tensor<32x8xbf16>) -> tensor<16x8xf32> {\n"
        "  %0 = xt.matmul(%a, %b) : tensor<16x32xbf16>, tensor<32x8xbf16> -> tensor<16x8xf32>\n"
        "  return %0 : tensor<16x8xf32>\n}"
    )
    assert "xt.matmul" in xt._module_asm(xt.parse(text))
    with pytest.raises(ValueError, match="requires matching element types or i8 inputs"):
        xt.parse(text.replace("tensor<32x8xbf16>", "tensor<32x8xf16>"))


# -- passes --------------------------------------------------------------------------


def test_serialize_order_and_constants():
    m = xt.parse(SERIAL.replace("SHARED", ""))
    xt.xt_serialize(m)
    text = xt._module_asm(m)
    consts = [int(v) for v in re.findall(r"arith.constant (\d+) : i32", text)]
    # z -> y -> x order, three constants (x, y, z) per block
    assert consts == [0, 0, 0, 1, 0, 0, 0, 1, 0, 1, 1, 0]
    assert text.count("xt.load(") == 4 and text.count("xt.store(") == 4


@pytest.mark.parametrize("shared,grid,loads", [(1, (2, 2, 1), 2), (2, (2, 2, 2), 2), (2, (3, 2, 1), 1), (0, (2, 2, 1), 4)])
def test_serialize_shared_reuse(shared, grid, loads):
    src = SERIAL.replace("SHARED", f"{{shared = {shared} : i64}}").replace(
        "array<i32: 2, 2, 1>", "array<i32: %d, %d, %d>" % grid
    )
    m = xt.parse(src)
    xt.xt_serialize(m)
    text = xt._module_asm(m)
    assert text.count("xt.load(") == loads
    assert text.count("xt.store(") == grid[0] * grid[1] * grid[2]


@pytest.mark.parametrize(
    "text,msg",
    [
        (SERIAL.replace("SHARED", "").replace(" attributes {xt.grid = array<i32: 2, 2, 1>}", ""),
         "xt-serialize requires func.func xt.grid attribute"),
        ("func.func @f(%a: memref<4xf32>) -> i32 attributes {xt.grid = array<i32: 1, 1, 1>} {\n"
         "  %b:3 = xt.get_tile_block_id : i32, i32, i32\n  func.return %b#0 : i32\n}",
         "xt-serialize only supports void functions"),
        ("func.func @f(%c: i1) attributes {xt.grid = array<i32: 1, 1, 1>} {\n  cf.cond_br %c, ^a, ^b\n"
         "^a:\n  func.return\n^b:\n  func.return\n}",
         "xt-serialize only supports single-block functions"),
    ],
)
def test_serialize_errors(text, msg):
    m = xt.parse(text)
    with pytest.raises(RuntimeError, match=msg):
        xt.xt_serialize(m)


def test_canonicalize_folds_zero():
    text = (
        "func.func @f(%a: tensor<16x16xf32>) -> tensor<16x16xf32> {\n"
        "  %z = arith.constant dense<0.0> : tensor<16x16xf32>\n"
        "  %0 = xt.add(%z, %a) : tensor<16x16xf32>, tensor<16x16xf32> -> tensor<16x16xf32>\n"
        "  %1 = xt.sub(%0, %z) : tensor<16x16xf32>, tensor<16x16xf32> -> tensor<16x16xf32>\n"
        "  return %1 : tensor<16x16xf32>\n}"
    )
    m = xt.parse(text)
    xt.canonicalize(m)
    out = xt._module_asm(m)
    assert "xt.add" not in out and "xt.sub" not in out and "arith.constant" not in out
    assert "return %arg0 : tensor<16x16xf32>" in out


def test_canonicalize_keeps_nonzero_and_side_effects():
    text = (
        "func.func @f(%a: memref<16x16xf32>) {\n  %c = arith.constant 0 : i32\n"
        "  %z = arith.constant dense<1.0> : tensor<16x16xf32>\n"
        "  %0 = xt.load(%a, %c, %c) : (memref<16x16xf32>, i32, i32) -> tensor<16x16xf32>\n"
        "  %1 = xt.sub(%0, %z) : tensor<16x16xf32>, tensor<16x16xf32> -> tensor<16x16xf32>\n"
        "  xt.store(%1, %a, %c, %c) : (tensor<16x16xf32>, memref<16x16xf32>, i32, i32) -> ()\n"
        "  func.return\n}"
    )
    m = xt.parse(text)
    xt.canonicalize(m)
    out = xt._module_asm(m)
    assert "xt.sub" in out and "xt.load" in out and "xt.store" in out


# -- xt-opt ----------------------------------------------------------------------------


def test_xt_opt_cli():
    rc, out, err = xt_opt(["--xt-serialize"], SERIAL.replace("SHARED", ""))
    assert rc == 0 and "xt.get_tile_block_id" not in out
    rc, out, err = xt_opt(["--split-input-file"], "func.func @a() {\n  func.return\n}\n// -----\nfunc.func @b( {\n")
    assert rc == 1 and "@a" in out and "error:" in err


def _run_line(path: Path) -> str:
    for line in path.read_text().splitlines():
        if line.startswith("// RUN:"):
            return line[len("// RUN:"):].strip()
    raise AssertionError("no RUN line")


@pytest.mark.skipif(not REF_TESTS.exists(), reason="reference tree not mounted (build container only)")
@pytest.mark.parametrize("name", ["parse", "serialize", "canonicalize", "invalid", "serialize_invalid", "to_nova"])
def test_reference_lit_file(name, tmp_path):
    """Run the reference's own lit test through this xt-opt and FileCheck."""
    path = REF_TESTS / f"{name}.mlir"
    run = _run_line(path).replace("%s", str(path))
    m = re.match(r"(not )?xt-opt (.*?) (?:2>&1 )?\| FileCheck (.*)$", run)
    assert m, run
    negate, opt_args, fc_args = m.group(1), m.group(2).split(), m.group(3).split()
    p = subprocess.run([str(XT_OPT), *opt_args], capture_output=True, text=True, timeout=60)
    output = p.stdout + (p.stderr if "2>&1" in run else "")
    assert (p.returncode != 0) if negate else (p.returncode == 0), p.stderr
    fc = subprocess.run([FILECHECK, *fc_args], input=output, capture_output=True, text=True, timeout=60)
    assert fc.returncode == 0, fc.stderr


# -- C ABI ----------------------------------------------------------------------------------


def _declared_functions() -> list[str]:
    header = (ROOT / "include" / "xtile_amd.h").read_text()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    return sorted(set(re.findall(r"\b(xt_[a-z_]+)\s*\(", header)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_xtile.LIB_FILE)
    declared = _declared_functions()
    assert "xt_gpu_run" in declared and "xt_module_parse" in declared
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_xtile.SIGNATURES)


def test_ceiling_library_exports_every_declared_symbol():
    """libxt_ceiling.so (bench.py's measurement kernels) exports what
    include/xt_ceiling.h declares, and refuses bad arguments on the host."""
    header = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "xt_ceiling.h").read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(xt_[a-z_]+)\s*\(", header)))
    assert declared == ["xt_ceiling_copy", "xt_ceiling_hold", "xt_ceiling_mfma", "xt_ceiling_noop"]
    import bench

    lib = bench._ceiling_lib()
    for name in declared:
        assert hasattr(lib, name), name
    # misaligned sizes, empty grids and unknown kinds are refused before any launch
    assert lib.xt_ceiling_copy(0x1000, 0x2000, 15, None) != 0
    assert lib.xt_ceiling_noop(0, None) != 0
    assert lib.xt_ceiling_hold(0, None) != 0 and lib.xt_ceiling_hold(1000001, None) != 0
    assert bench.hold_us(20, eager=True) == 1300 and bench.hold_us(10**4, eager=True) == 5000
    assert bench.hold_us(2000, eager=False) == 2500 and bench.hold_us(10**7, eager=False) == 10**6
    assert lib.xt_ceiling_mfma(0x1000, 0x2000, 1, 1, 7, None) != 0


def test_bench_checks_tell_results_apart():
    import bench

    x = np.array([1.0, 2.0, 3.0], np.float32)
    assert bench.compare("exact", 0.0, x, x.copy(), "f32")[0]
    assert not bench.compare("exact", 0.0, x, x + np.float32(1e-7), "f32")[0]
    assert bench.compare("max_rel", 1e-5, x * np.float32(1 + 5e-6), x, "f32")[0]
    assert not bench.compare("max_rel", 1e-5, x * np.float32(1 + 5e-5), x, "f32")[0]
    assert not bench.compare("frob", 1e-3, x[::-1].copy(), x, "f32")[0]
    b = bench.bf16_bits(x)
    assert bench.compare("frob", 1e-3, b, b.copy(), "bf16")[0]


def test_version_string():
    assert "gfx950" in _xtile.version()


def test_signature_json():
    from xtile_amd import kernels as K

    sig = xt.signature(K.add(64, 128))
    assert sig["grid"] == [2, 2, 1]
    assert sig["args"][0] == {"kind": "memref", "dtype": "f32", "shape": [64, 128]}


def test_launch_rejects_bad_buffers_before_any_device_call():
    """Buffer checks happen on the host, before the HIP runtime is touched."""
    from xtile_amd import kernels as K

    m = K.add(64, 128)
    fake = [0x1000, 0x2000, 0x3000]
    with pytest.raises(ValueError, match="takes 3 buffers, got 2"):
        _xtile.launch(m, None, fake[:2], [32768, 32768])
    with pytest.raises(ValueError, match="needs 32768"):
        _xtile.launch(m, None, fake, [32768, 32768, 100])
    with pytest.raises(ValueError, match="is null"):
        _xtile.launch(m, None, [0x1000, 0, 0x3000], [32768] * 3)
