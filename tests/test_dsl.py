"""The tracing DSL: exact emitted text, validation errors, naming rules.

Exact text is pinned by tests/golden/dsl/*.mlir, written by the reference's own
tracer (tests/golden/make_dsl_golden.py).  Error behaviour mirrors
xtile/dsl.py's validation (message text and exception type).
"""

from __future__ import annotations

from pathlib import Path

import pytest

import xtile_amd as xt
from xtile_amd import dsl
from tests.golden.dsl_programs import programs

GOLDEN = Path(__file__).resolve().parent / "golden" / "dsl"


@pytest.mark.parametrize("name", sorted(programs(dsl).keys()))
def test_emitted_text_matches_reference_tracer(name):
    kernel, args, grid, db = programs(dsl)[name]
    text = dsl.convert(kernel, args=args, grid=grid, double_buffering=db, parse_module=lambda s: s)
    assert text + "\n" == (GOLDEN / f"{name}.mlir").read_text()


@pytest.mark.parametrize("name", sorted(programs(dsl).keys()))
def test_emitted_text_parses_and_displays_verbatim(name):
    kernel, args, grid, db = programs(dsl)[name]
    module = xt.convert(kernel, args=args, grid=grid, double_buffering=db)
    assert str(module) + "\n" == (GOLDEN / f"{name}.mlir").read_text()
    # the native printer round-trips through the parser
    printed = xt._module_asm(module)
    assert xt._module_asm(xt.parse(printed)) == printed


def test_serialize_returns_same_module_and_clears_display():
    kernel, args, grid, db = programs(dsl)["rowwise_softmax"]
    module = xt.convert(kernel, args=args, grid=grid, double_buffering=db)
    assert xt.xt_serialize(module) is module
    text = str(module)
    assert text.startswith("module {")
    assert "xt.get_tile_block_id" not in text
    assert text.count("xt.load(") == 2  # grid (2, 1, 1)


def test_truediv_is_mul_of_reciprocal():
    kernel, args, grid, db = programs(dsl)["divide_kernel"]
    text = str(xt.convert(kernel, args=args, grid=grid, double_buffering=db))
    assert "xt.reciprocal(" in text and "xt.mul(" in text and "xt.div" not in text


# -- extension dtypes ---------------------------------------------------------


def test_f16_matmul_gives_f32():
    @xt.kernel
    def mm(a, b, c):
        x = xt.load(a, index=(xt.bid(0), 0), shape=(64, 64))
        y = xt.load(b, index=(0, xt.bid(1)), shape=(64, 64), shared=1)
        xt.store(c, index=(xt.bid(0), xt.bid(1)), tile=xt.matmul(x, y))

    m = xt.convert(
        mm,
        args=(
            xt.Array((128, 64), xt.float16),
            xt.Array((64, 128), xt.float16),
            xt.Array((128, 128), xt.float32),
        ),
        grid=(2, 2, 1),
    )
    assert "tensor<64x64xf16>, tensor<64x64xf16> -> tensor<64x64xf32>" in str(m)
    assert xt.plan(m)["kernel"].startswith("gemm f16->f32")


def test_bf16_load_conv2d_gives_f32():
    @xt.kernel
    def cv(x, f, y):
        w = xt.load(f, index=(0, 0, 0, 0), shape=(3, 3, 32, 16), shared=2)
        t = xt.load_conv2d(x, w, index=(0, xt.bid(0), 0, 0), shape=(1, 4, 8, 16),
                           pad=(1, 1, 1, 1), stride=(1, 1), dilation=(1, 1))
        xt.store(y, index=(0, xt.bid(0), 0, 0), tile=t)

    m = xt.convert(
        cv,
        args=(
            xt.Array((1, 8, 8, 32), xt.bfloat16),
            xt.Array((3, 3, 32, 16), xt.bfloat16),
            xt.Array((1, 8, 8, 16), xt.float32),
        ),
        grid=(2, 1, 1),
    )
    assert "-> tensor<1x4x8x16xf32>" in str(m)


def test_mixed_dtype_matmul_rejected():
    @xt.kernel
    def mm(a, b, c):
        xt.store(c, index=(0, 0), tile=xt.matmul(xt.load(a, index=(0, 0), shape=(4, 4)),
                                                 xt.load(b, index=(0, 0), shape=(4, 4))))

    with pytest.raises(TypeError, match="matching dtypes"):
        xt.convert(mm, args=(xt.Array((4, 4), xt.float16), xt.Array((4, 4), xt.bfloat16),
                             xt.Array((4, 4), xt.float32)), grid=(1, 1, 1))


# -- validation (xtile/dsl.py) -------------------------------------------------


def _one(body, *arrays, grid=(1, 1, 1)):
    """Trace `body` as a kernel over `arrays` (convert needs a fixed-arity signature)."""
    names = ", ".join(f"a{i}" for i in range(len(arrays)))
    ns = {"body": body}
    exec(f"def k({names}):\n    body({names})", ns)
    return xt.convert(xt.kernel(ns["k"]), args=arrays, grid=grid)


F = xt.Array((16, 16), xt.float32)


@pytest.mark.parametrize(
    "grid", [(1, 1), (0, 1, 1), (1, -1, 1), (1.0, 1, 1), [1, 1, 1]]
)
def test_bad_grid(grid):
    with pytest.raises(ValueError, match="grid must be a 3-tuple of positive integers"):
        _one(lambda a: None, F, grid=grid)


def test_arg_count_and_types():
    @xt.kernel
    def k(a, b):
        pass

    with pytest.raises(ValueError, match="convert args must match the kernel signature"):
        xt.convert(k, args=(F,), grid=(1, 1, 1))
    with pytest.raises(TypeError, match="xt.Array values or integers"):
        xt.convert(k, args=(F, 1.5), grid=(1, 1, 1))
    with pytest.raises(TypeError, match="decorated with @xt.kernel"):
        xt.convert(lambda a: None, args=(F,), grid=(1, 1, 1))


def test_kernel_must_return_none():
    @xt.kernel
    def k(a):
        return 1

    with pytest.raises(ValueError, match="must not return a value"):
        xt.convert(k, args=(F,), grid=(1, 1, 1))


def test_ops_outside_trace():
    with pytest.raises(RuntimeError, match="xt.bid may only be used while converting a kernel"):
        xt.bid(0)
    with pytest.raises(RuntimeError, match="xt.exp may only be used"):
        xt.exp(None)


def test_array_validation():
    with pytest.raises(TypeError):
        xt.Array((), xt.float32)
    with pytest.raises(TypeError):
        xt.Array((4, 0), xt.float32)
    with pytest.raises(TypeError):
        xt.Array((4, 4), "f32")


@pytest.mark.parametrize(
    "body,exc,msg",
    [
        (lambda a: xt.bid(3), ValueError, "dimensions 0, 1, and 2"),
        (lambda a: xt.load(a, index=(0,), shape=(16, 16)), ValueError, "index rank"),
        (lambda a: xt.load(a, index=(0, 0), shape=(16,)), ValueError, "shape rank"),
        (lambda a: xt.load(a, index=(0, 0), shape=(16, 16), shared=3), ValueError, "shared must be"),
        (lambda a: xt.load(a, index=(0, 0.5), shape=(16, 16)), TypeError, "index values"),
        (lambda a: xt.load(a, index=[0, 0], shape=(16, 16)), TypeError, "index must be"),
        (lambda a: xt.load(a, index=(0, 0), shape=(16, 0)), TypeError, "shape must be"),
        (lambda a: xt.load(1, index=(0, 0), shape=(16, 16)), TypeError, "kernel arguments"),
        (lambda a: xt.store(a, index=(0, 0), tile=1), TypeError, "expects a tensor value"),
        (
            lambda a: xt.add(xt.load(a, index=(0, 0), shape=(16, 16)), xt.load(a, index=(0, 0), shape=(8, 16))),
            ValueError,
            "broadcast-compatible",
        ),
        (
            lambda a: xt.sub(xt.load(a, index=(0, 0), shape=(16, 1)), xt.load(a, index=(0, 0), shape=(16, 16))),
            ValueError,
            "broadcast-compatible",
        ),
        (lambda a: xt.max(xt.reshape(xt.load(a, index=(0, 0), shape=(16, 16)), shape=(256,))), ValueError, "rank-2"),
        (lambda a: xt.sum(xt.load(a, index=(0, 0), shape=(16, 16)), axis=2), ValueError, "axis must be in range"),
        (lambda a: xt.reshape(xt.load(a, index=(0, 0), shape=(16, 16)), shape=(3, 5)), ValueError, "same number"),
        (lambda a: xt.transpose(xt.load(a, index=(0, 0), shape=(16, 16))), ValueError, "rank-3"),
        (lambda a: xt.astype(xt.load(a, index=(0, 0), shape=(16, 16)), dtype=xt.float16), TypeError, "int8<->float32"),
        (lambda a: dsl.truediv(xt.load(a, index=(0, 0), shape=(16, 16)), 2.0), TypeError, "tensor rhs"),
    ],
)
def test_validation_errors(body, exc, msg):
    with pytest.raises(exc, match=msg):
        _one(body, F)


def test_matmul_and_mma_validation():
    i8 = xt.Array((16, 16), xt.int8)
    with pytest.raises(ValueError, match="inner dimension"):
        _one(lambda a: xt.matmul(xt.load(a, index=(0, 0), shape=(16, 8)), xt.load(a, index=(0, 0), shape=(4, 16))), i8)
    with pytest.raises(TypeError, match="int8 lhs and rhs"):
        _one(
            lambda a: xt.mma(
                xt.load(a, index=(0, 0), shape=(4, 4)),
                xt.load(a, index=(0, 0), shape=(4, 4)),
                xt.load(a, index=(0, 0), shape=(4, 4)),
            ),
            F,
        )


def test_load_conv2d_validation():
    src = xt.Array((1, 8, 8, 32), xt.int8)
    filt = xt.Array((3, 3, 16, 16), xt.int8)
    out = xt.Array((1, 8, 8, 16), xt.float32)

    def body(x, f, y):
        w = xt.load(f, index=(0, 0, 0, 0), shape=(3, 3, 16, 16))
        xt.load_conv2d(x, w, index=(0, 0, 0, 0), shape=(1, 8, 8, 16), pad=(1, 1, 1, 1),
                       stride=(1, 1), dilation=(1, 1))

    with pytest.raises(ValueError, match="channel dimensions to match"):
        _one(body, src, filt, out)

    def bad_stride(x, f, y):
        w = xt.load(f, index=(0, 0, 0, 0), shape=(3, 3, 16, 16))
        xt.load_conv2d(x, w, index=(0, 0, 0, 0), shape=(1, 8, 8, 16), pad=(1, 1, 1, 1),
                       stride=(0, 1), dilation=(1, 1))

    with pytest.raises(ValueError, match="stride values must be positive"):
        _one(bad_stride, src, filt, out)


def test_arg_naming_rules():
    @xt.kernel
    def k(p, q, r, s):
        t = xt.load(p, index=(0, 0), shape=(16, 16))
        u = xt.load(q, index=(0, 0), shape=(16, 16))
        xt.store(q, index=(0, 0), tile=t)      # q loaded and stored: keeps its name
        xt.store(r, index=(0, 0), tile=u)
        xt.store(s, index=(0, 0), tile=u)

    text = str(xt.convert(k, args=(F, F, F, F), grid=(1, 1, 1)))
    assert "@k(%input: memref<16x16xf32>, %q: memref<16x16xf32>, %output: memref<16x16xf32>, %output2:" in text
