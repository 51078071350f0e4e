"""The package serves the reference's interface on the PKM path (CPU only).

tests/golden/reference_interface.json was written from the reference's source
text with `ast` by tests/golden/make_interface_golden.py: the package-relative
imports of modeling_qwen3pkm.py and every top-level function / class of the
modules on the path, with parameter names and default values. Checked here:
  * every import of modeling_qwen3pkm.py (:20-24) resolves inside modelos_amd,
    so the modeling file placed in the package imports unchanged;
  * every reference function and class exists under the same module path with
    the same parameters, in order, and the same defaults; every reference
    method exists with the same parameters.
Deliberately absent (ABSENT below): the Triton kernels (replaced by HIP
kernels behind the C ABI), the CPU fallback backward (this path has no CPU
fallback) and ColwiseEmbeddingBag (multi-GPU tensor parallelism).
"""
from __future__ import annotations

import ast
import importlib
import inspect
import json
from pathlib import Path

import pytest

IFACE = json.loads((Path(__file__).resolve().parent / "golden" / "reference_interface.json").read_text())

ABSENT = {
    ("fwpkm.xformer_embeddingbag_legacy", "_embedding_bag_bw_native"): "CPU fallback; no CPU path here",
    ("pkm.colwise_embedding_bag", "ColwiseEmbeddingBag"): "multi-GPU tensor-parallel style; one GPU here",
}


def _entries():
    for mod, entries in IFACE["modules"].items():
        for name, e in entries.items():
            yield mod, name, e


def _is_triton_kernel(e) -> bool:
    return any("triton.jit" in d for d in e.get("decorators", []))


def _literal(src):
    try:
        return True, ast.literal_eval(src)
    except (ValueError, SyntaxError):
        return False, None


def _check_params(ours: inspect.Signature, ref_params, what: str, skip_self: bool):
    ref = ref_params[1:] if skip_self and ref_params and ref_params[0][0] in ("self", "ctx", "cls") else ref_params
    params = list(ours.parameters.values())
    if params and params[0].name in ("self", "ctx", "cls") and (not ref or ref[0][0] != params[0].name):
        params = params[1:]
    names = [("*" if p.kind == p.VAR_POSITIONAL else "**" if p.kind == p.VAR_KEYWORD else "") + p.name
             for p in params]
    assert names == [r[0] for r in ref], f"{what}: parameters {names} != reference {[r[0] for r in ref]}"
    for p, (rname, rdefault) in zip(params, ref):
        if rdefault is None:
            assert p.default is inspect.Parameter.empty or p.kind in (p.VAR_POSITIONAL, p.VAR_KEYWORD), \
                f"{what}: {rname} has a default here but not in the reference"
            continue
        ok, value = _literal(rdefault)
        if ok:
            assert p.default == value and type(p.default) is type(value), \
                f"{what}: default of {rname} is {p.default!r}, reference {rdefault}"


def test_modeling_imports_resolve():
    for module, names in IFACE["modeling_imports"]:
        mod = importlib.import_module("modelos_amd." + module)
        for name in names:
            assert hasattr(mod, name), f"modelos_amd.{module} lacks {name} (modeling_qwen3pkm.py imports it)"


@pytest.mark.parametrize("mod,name,e", [pytest.param(*t, id=f"{t[0]}.{t[1]}") for t in _entries()])
def test_reference_name_present_with_signature(mod, name, e):
    if _is_triton_kernel(e):
        pytest.skip("Triton kernel: replaced by the HIP kernels behind include/pkm_hip.h")
    if (mod, name) in ABSENT:
        assert not hasattr(importlib.import_module("modelos_amd." + mod), name)
        pytest.skip(ABSENT[(mod, name)])
    obj = getattr(importlib.import_module("modelos_amd." + mod), name, None)
    assert obj is not None, f"modelos_amd.{mod}.{name} missing"
    if e["kind"] == "function":
        _check_params(inspect.signature(obj), e["params"], f"{mod}.{name}", skip_self=False)
        return
    assert inspect.isclass(obj)
    for meth, params in e["methods"].items():
        fn = inspect.getattr_static(obj, meth, None)
        assert fn is not None, f"{mod}.{name}.{meth} missing"
        fn = fn.__func__ if isinstance(fn, (staticmethod, classmethod)) else fn
        _check_params(inspect.signature(fn), params, f"{mod}.{name}.{meth}", skip_self=True)


def test_config_fields_and_defaults():
    from modelos_amd.configuration_qwen3pkm import Qwen3PKMConfig

    cfg = Qwen3PKMConfig(num_hidden_layers=28, pkm_layers=[8, 20], fwpkm_layers=[3])
    params = IFACE["modules"]["configuration_qwen3pkm"]["Qwen3PKMConfig"]["methods"]["__init__"]
    for pname, default in params:
        if pname in ("self", "**kwargs"):
            continue
        ok, value = _literal(default)
        if pname == "pkm_layers":
            assert cfg.pkm_layers == [8, 20]
        elif pname == "fwpkm_layers":
            assert cfg.fwpkm_layers == [3]
        elif ok:
            assert getattr(cfg, pname) == value, pname
    assert cfg.model_type == "qwen3_pkm" and cfg.num_fwpkm_layers == 1
    with pytest.raises(ValueError):
        Qwen3PKMConfig(num_hidden_layers=4, pkm_layers=[4])
    with pytest.raises(NotImplementedError):
        Qwen3PKMConfig(fwpkm_query_src="output")
