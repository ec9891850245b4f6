"""Write tests/golden/dsl/*.mlir: the reference tracer's text for each program
of tests/golden/dsl_programs.py.

Runs only in the build container, where the reference tree is mounted at
/root/reference.  The reference's xtile/dsl.py is pure Python; it is loaded by
file path (its package __init__ needs the native _xtile module, which cannot be
built here) and its `convert` is given an identity `parse_module`, so the
emitted text is captured verbatim.  Nothing from the reference is copied into
this repository except these output texts.

    python tests/golden/make_dsl_golden.py
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF_DSL = Path("/root/reference/xtile/dsl.py")


def main() -> int:
    if not REF_DSL.exists():
        print("reference tree not mounted; nothing to do", file=sys.stderr)
        return 1
    spec = importlib.util.spec_from_file_location("reference_xtile_dsl", REF_DSL)
    ref = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = ref  # dataclasses look the module up while executing it
    spec.loader.exec_module(ref)
    sys.path.insert(0, str(HERE))
    from dsl_programs import programs

    out_dir = HERE / "dsl"
    out_dir.mkdir(exist_ok=True)
    for name, (kernel, args, grid, db) in programs(ref).items():
        text = ref.convert(kernel, args=args, grid=grid, double_buffering=db, parse_module=lambda s: s)
        (out_dir / f"{name}.mlir").write_text(text + "\n")
        print(f"wrote {name}.mlir")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
