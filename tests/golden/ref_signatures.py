"""Write the reference's public call signatures for the verification path to
ref_signatures.json, reading its source text with ``ast`` (nothing of the
reference is imported or run).

Recorded per function: the parameter names in order, which have defaults (and
the literal default where it is a constant), keyword-only parameters, and
whether it is a method (``self``) or a staticmethod. Run from the repository
root with the reference checked out at /root/reference:

    python tests/golden/ref_signatures.py
"""

from __future__ import annotations

import ast
import json
from pathlib import Path

REF = Path("/root/reference/src/pe")
OUT = Path(__file__).resolve().parent / "ref_signatures.json"

# (file, class or None, function)
WANTED = [
    ("target.py", "TargetModel", "forward_cached"),
    ("target.py", "TargetModel", "forward"),
    ("target.py", "TargetModel", "make_cache"),
    ("target.py", "TargetModel", "gather_cache"),
    ("target.py", "TargetModel", "get_input_embeddings"),
    ("target.py", "TargetModel", "get_lm_head"),
    ("target.py", "TargetModel", "get_final_norm"),
    ("masks.py", None, "to_additive_bias"),
    ("masks.py", None, "tree_depths"),
    ("masks.py", None, "tree_allow_mask"),
    ("masks.py", None, "tree_position_ids"),
    ("decode/verify.py", None, "accept_tree_cached"),
    ("decode/verify.py", None, "accept_tree_greedy"),
    ("decode/tree.py", None, "propose_tree"),
]


def _signature(fn: ast.FunctionDef) -> dict:
    a = fn.args
    pos = [p.arg for p in a.posonlyargs + a.args]
    defaults = {}
    for name, d in zip(pos[len(pos) - len(a.defaults):], a.defaults):
        defaults[name] = d.value if isinstance(d, ast.Constant) else ast.unparse(d)
    kwonly = [p.arg for p in a.kwonlyargs]
    for p, d in zip(a.kwonlyargs, a.kw_defaults):
        if d is not None:
            defaults[p.arg] = d.value if isinstance(d, ast.Constant) else ast.unparse(d)
    decos = [ast.unparse(d) for d in fn.decorator_list]
    return {"params": pos, "kwonly": kwonly, "defaults": defaults, "staticmethod": "staticmethod" in decos,
            "line": fn.lineno}


def main() -> None:
    out = {}
    for rel, cls, name in WANTED:
        tree = ast.parse((REF / rel).read_text())
        scope = tree.body
        if cls is not None:
            scope = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == cls).body
        fn = next(n for n in scope if isinstance(n, ast.FunctionDef) and n.name == name)
        key = f"{cls}.{name}" if cls else name
        out[key] = {"file": f"src/pe/{rel}", **_signature(fn)}
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({len(out)} signatures)")


if __name__ == "__main__":
    main()
