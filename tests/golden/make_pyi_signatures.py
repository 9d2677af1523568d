"""Writes tests/golden/cache_ops_pyi_signatures.json: the parameter names,
kinds, defaults and annotations of the reference's `daric.cache_ops` API as
its type stub declares them (daric/cache_ops.pyi:6-53).

The stub is parsed as text with `ast`; nothing of the reference is imported
or run. Only the extracted names and defaults are committed.

    python tests/golden/make_pyi_signatures.py [/root/reference]
"""
from __future__ import annotations

import ast
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "cache_ops_pyi_signatures.json")


def params(fn: ast.FunctionDef) -> list:
    a = fn.args
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    out = []
    for arg, d in zip(pos, defaults):
        out.append({
            "name": arg.arg,
            "kind": "POSITIONAL_OR_KEYWORD",
            "default": None if d is None else ast.literal_eval(d),
            "has_default": d is not None,
            "annotation": None if arg.annotation is None else ast.unparse(arg.annotation),
        })
    for arg, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append({"name": arg.arg, "kind": "KEYWORD_ONLY",
                    "default": None if d is None else ast.literal_eval(d), "has_default": d is not None,
                    "annotation": None if arg.annotation is None else ast.unparse(arg.annotation)})
    return out


def main(ref_root: str) -> None:
    path = os.path.join(ref_root, "daric", "cache_ops.pyi")
    tree = ast.parse(open(path).read())
    sigs = {}
    for node in tree.body:
        if isinstance(node, ast.FunctionDef):
            sigs[node.name] = {"params": params(node), "returns": ast.unparse(node.returns)}
        elif isinstance(node, ast.ClassDef):
            for m in node.body:
                if isinstance(m, ast.FunctionDef):
                    sigs[f"{node.name}.{m.name}"] = {"params": params(m), "returns": ast.unparse(m.returns)}
    doc = {"source": "daric/cache_ops.pyi (parsed with ast)", "signatures": sigs}
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT}: {len(sigs)} signatures")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
