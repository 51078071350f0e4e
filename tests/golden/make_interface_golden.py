"""Writes tests/golden/reference_interface.json: the reference's public
interface on the PKM path, read from its source text with `ast` (nothing is
imported or run).

Run in a checkout that has the reference at REFERENCE (default
/root/reference):  python tests/golden/make_interface_golden.py

Recorded:
  * "modeling_imports": the package-relative imports of
    modeling_qwen3pkm.py (module, names), which a drop-in package must serve;
  * "modules": for each module on the path, its top-level functions and
    classes: parameter names with default-value source text, and for classes
    the __init__ and every method signature.
configuration_qwen3pkm.py does not parse as a whole (an unterminated string
at :99); its class header and __init__ signature are parsed from the text
before the first statement of the __init__ body.
"""
from __future__ import annotations

import ast
import json
import os
from pathlib import Path

REFERENCE = Path(os.environ.get("REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent / "reference_interface.json"

MODULES = [
    "configuration_qwen3pkm",
    "pkm/memory",
    "pkm/xformer_embeddingbag",
    "pkm/colwise_embedding_bag",
    "fwpkm/fwpkm",
    "fwpkm/fwmlp",
    "fwpkm/xformer_embeddingbag_grad_wrapper",
    "fwpkm/xformer_embeddingbag_legacy",
]


def _params(fn: ast.FunctionDef):
    a = fn.args
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + [ast.unparse(d) for d in a.defaults]
    out = [[p.arg, d] for p, d in zip(pos, defaults)]
    if a.vararg:
        out.append(["*" + a.vararg.arg, None])
    for p, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append([p.arg, ast.unparse(d) if d is not None else None])
    if a.kwarg:
        out.append(["**" + a.kwarg.arg, None])
    return out


def _decorators(node):
    return [ast.unparse(d) for d in node.decorator_list]


def _module_entries(tree: ast.Module):
    entries = {}
    for node in tree.body:
        if isinstance(node, ast.FunctionDef):
            entries[node.name] = {"kind": "function", "params": _params(node), "decorators": _decorators(node)}
        elif isinstance(node, ast.ClassDef):
            methods = {m.name: _params(m) for m in node.body if isinstance(m, ast.FunctionDef)}
            entries[node.name] = {"kind": "class", "bases": [ast.unparse(b) for b in node.bases],
                                  "methods": methods}
    return entries


def _config_entries(text: str):
    # keep the text up to the end of the __init__ signature, then close the body
    head = text[: text.index("super().__init__(**kwargs)")]
    tree = ast.parse(head + "pass\n")
    return _module_entries(tree)


def main():
    modeling = ast.parse((REFERENCE / "modeling_qwen3pkm.py").read_text())
    imports = [[node.module, [a.name for a in node.names]]
               for node in modeling.body if isinstance(node, ast.ImportFrom) and node.level >= 1]
    modules = {}
    for mod in MODULES:
        text = (REFERENCE / f"{mod}.py").read_text()
        modules[mod.replace("/", ".")] = (_config_entries(text) if mod == "configuration_qwen3pkm"
                                          else _module_entries(ast.parse(text)))
    OUT.write_text(json.dumps({"modeling_imports": imports, "modules": modules}, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
