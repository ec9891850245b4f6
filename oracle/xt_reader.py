"""TEST INFRASTRUCTURE: an independent reader of xt function text.

Deliberately separate from the product's C++ parser (xtile_amd/csrc/ir.cpp):
a regex reader for the line-per-op form the DSL emits (xtile/dsl.py:490-620)
and the printer writes.  It returns a plain description of one function that
the oracle executors consume.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

_TYPE = re.compile(r"(tensor|memref)<((?:\d+x)*)(f32|f16|bf16|i8|i32)>")
_FUNC = re.compile(
    r"func\.func\s+@([\w$.-]+)\s*\((.*?)\)\s*(?:attributes\s*\{(.*?)\})?\s*\{", re.S
)
_GRID = re.compile(r"xt\.grid\s*=\s*array<i32:\s*(\d+)\s*,\s*(\d+)\s*,\s*(\d+)\s*>")


@dataclass
class TType:
    kind: str  # "tensor" | "memref"
    shape: tuple[int, ...]
    dtype: str


def parse_type(text: str) -> TType:
    m = _TYPE.search(text)
    if not m:
        raise ValueError(f"cannot read type from {text!r}")
    dims = tuple(int(d) for d in m.group(2).split("x") if d)
    return TType(m.group(1), dims, m.group(3))


@dataclass
class ROp:
    name: str
    results: list[str]
    operands: list[str]
    attrs: dict[str, object]
    operand_types: list[TType]
    result_type: TType | None


@dataclass
class RFunc:
    name: str
    args: list[tuple[str, TType]]
    grid: tuple[int, int, int]
    ops: list[ROp] = field(default_factory=list)


def _split_top(s: str) -> list[str]:
    """Split on commas not nested in <>, (), [] or {}."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "<([{":
            depth += 1
        elif ch in ">)]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _attrs(text: str) -> dict[str, object]:
    out: dict[str, object] = {}
    for item in _split_top(text):
        if "=" not in item:
            out[item.strip()] = True
            continue
        k, v = item.split("=", 1)
        k, v = k.strip(), v.strip()
        m = re.match(r"array<i\d+:\s*(.*)>", v)
        if m:
            out[k] = tuple(int(x) for x in m.group(1).split(",") if x.strip())
            continue
        m = re.match(r"\[(.*)\]", v)
        if m:
            out[k] = tuple(int(x) for x in m.group(1).split(",") if x.strip())
            continue
        m = re.match(r"(-?\d+)\s*:", v)
        if m:
            out[k] = int(m.group(1))
            continue
        out[k] = v
    return out


def read_function(text: str, name: str | None = None) -> RFunc:
    funcs = []
    for m in _FUNC.finditer(text):
        fname, args_text, attrs_text = m.group(1), m.group(2), m.group(3) or ""
        g = _GRID.search(attrs_text)
        grid = tuple(int(x) for x in g.groups()) if g else (1, 1, 1)
        args = []
        for a in _split_top(args_text):
            an, at = a.split(":", 1)
            args.append((an.strip(), parse_type(at)))
        # body: from the opening brace to the matching close
        start = m.end()
        depth, pos = 1, start
        while depth and pos < len(text):
            if text[pos] == "{":
                depth += 1
            elif text[pos] == "}":
                depth -= 1
            pos += 1
        body = text[start : pos - 1]
        funcs.append((fname, args, grid, body))
    if not funcs:
        raise ValueError("no func.func found")
    if name is None:
        if len(funcs) != 1:
            raise ValueError("several functions; name one")
        chosen = funcs[0]
    else:
        chosen = next(f for f in funcs if f[0] == name)
    fname, args, grid, body = chosen
    fn = RFunc(fname, args, grid)
    for raw in body.splitlines():
        line = raw.strip()
        if not line or line.startswith("//"):
            continue
        results: list[str] = []
        m = re.match(r"^(%[^=]*?)\s*=\s*(.*)$", line)
        rest = line
        if m and not line.startswith("xt.store"):
            lhs, rest = m.group(1), m.group(2)
            for r in _split_top(lhs):
                r = r.strip()
                cm = re.match(r"(%[\w$.-]+):(\d+)$", r)
                if cm:
                    results.extend(f"{cm.group(1)}#{i}" for i in range(int(cm.group(2))))
                else:
                    results.append(r)
        opm = re.match(r"([\w.]+)(.*)$", rest)
        if not opm:
            raise ValueError(f"cannot read op from {line!r}")
        opname, tail = opm.group(1), opm.group(2).strip()
        if opname in ("func.return", "return"):
            continue
        if opname == "xt.get_tile_block_id":
            fn.ops.append(ROp(opname, results, [], {}, [], None))
            continue
        if opname == "arith.constant":
            cm = re.match(r"(-?\d+)\s*:\s*(i32|index)", tail)
            if not cm:
                raise ValueError(f"unsupported constant {line!r}")
            fn.ops.append(ROp(opname, results, [], {"value": int(cm.group(1))}, [], None))
            continue
        pm = re.match(r"\((.*?)\)\s*(.*)$", tail)
        if not pm:
            raise ValueError(f"cannot read operands of {line!r}")
        operands = [o.strip() for o in pm.group(1).split(",") if o.strip()]
        tail = pm.group(2)
        attrs: dict[str, object] = {}
        am = re.match(r"\{(.*?)\}\s*(.*)$", tail)
        if am:
            attrs = _attrs(am.group(1))
            tail = am.group(2)
        if not tail.startswith(":"):
            raise ValueError(f"missing types in {line!r}")
        sig = tail[1:].strip()
        ins_text, _, out_text = sig.rpartition("->")
        ins_text = ins_text.strip()
        if ins_text.startswith("(") and ins_text.endswith(")"):
            ins_text = ins_text[1:-1]
        operand_types = [
            parse_type(t) if ("tensor" in t or "memref" in t) else TType("scalar", (), t.strip())
            for t in _split_top(ins_text)
        ]
        out_text = out_text.strip()
        result_type = None if out_text == "()" else parse_type(out_text)
        fn.ops.append(ROp(opname, results, operands, attrs, operand_types, result_type))
    return fn
