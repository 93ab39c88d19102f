"""Write reference_signatures.json: the unified-API signatures of the
reference's golden implementations, read from their source text.

For each kernel directory of this family, ViperBench/<kernel>/pytorch_impl.py is
parsed with ``ast`` (never imported or executed) and every top-level function
the unified API names is recorded as its parameter names, kinds and default
values (as Python literals).  The fixture is data -- names and defaults -- and
lets ``tests/test_hip_impl_api.py`` check the hip_impl modules against the
reference's own text rather than against this repository's restatement.

    python tests/golden/make_ref_signatures.py [REFERENCE_ROOT]

REFERENCE_ROOT defaults to /root/reference (a read-only checkout of
tingxi-li/DSLPerfGap).
"""
from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

FUNCS = {
    "layer_norm": ["layer_norm"],
    "rms_norm": ["rms_norm"],
    "softmax": ["softmax"],
    "log_softmax": ["log_softmax"],
    "logsumexp": ["logsumexp"],
    "cross_entropy": ["cross_entropy_fwd", "cross_entropy_bwd"],
    "mean_reduction": ["mean_reduction"],
    "max_reduction": ["max_reduction"],
    "argmax": ["argmax"],
}
OUT = Path(__file__).resolve().parent / "reference_signatures.json"


def _params(fn: ast.FunctionDef) -> list[dict]:
    a = fn.args
    out = []
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    for arg, d in zip(pos, defaults):
        p = {"name": arg.arg, "kind": "positional_or_keyword"}
        if d is not None:
            p["default"] = ast.literal_eval(d)
        out.append(p)
    if a.vararg:
        out.append({"name": a.vararg.arg, "kind": "var_positional"})
    for arg, d in zip(a.kwonlyargs, a.kw_defaults):
        p = {"name": arg.arg, "kind": "keyword_only"}
        if d is not None:
            p["default"] = ast.literal_eval(d)
        out.append(p)
    if a.kwarg:
        out.append({"name": a.kwarg.arg, "kind": "var_keyword"})
    return out


def signatures(root: Path) -> dict:
    sigs = {}
    for kernel, names in FUNCS.items():
        rel = f"ViperBench/{kernel}/pytorch_impl.py"
        tree = ast.parse((root / rel).read_text(), filename=rel)
        defs = {n.name: n for n in tree.body if isinstance(n, ast.FunctionDef)}
        for name in names:
            fn = defs[name]
            sigs[name] = {"kernel": kernel, "file": f"{rel}:{fn.lineno}",
                          "params": _params(fn)}
    return sigs


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    root = Path(argv[0]) if argv else Path("/root/reference")
    OUT.write_text(json.dumps(signatures(root), indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
