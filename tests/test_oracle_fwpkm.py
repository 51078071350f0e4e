"""The fast-weight PKM oracle (oracle/fwpkm.py) against the reference's own
outputs (CPU only).

tests/golden/fwpkm_*.pt were written by the reference's
FastWeightProductKeyMemory (fwpkm/fwpkm.py) on the CPU by
tests/golden/make_fwpkm_golden.py: explicit parameters, inputs, upstream
gradient; outputs, indices, transformed scores, per-example losses, the
address loss, gradient norms, the fast weights after the call, and (for the
chunked forward) every outer gradient through the inner updates.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import pytest
import torch

from oracle import fwpkm as ofw
from tests.helpers import assert_rel_close

GOLDEN = Path(__file__).resolve().parent / "golden"
CHUNKED = ["idw_la0", "dot_la1"]


def load(case):
    return torch.load(GOLDEN / f"fwpkm_{case}.pt", weights_only=True)


@pytest.mark.parametrize("case", CHUNKED + ["stream"])
def test_golden_integrity(case):
    rec = load(case)
    assert rec["min_selection_gap"] >= 1e-4
    for call in rec["calls"]:
        c = call["inputs"]
        h = hashlib.sha256()
        for k in sorted(c):
            h.update(c[k].contiguous().numpy().tobytes())
        assert h.hexdigest() == call["sha256.inputs"]


@pytest.mark.parametrize("case", CHUNKED)
def test_oracle_chunked_matches_reference(case):
    rec = load(case)
    cfg = ofw.FwConfig.from_module_kwargs(rec["kwargs"])
    (call,) = rec["calls"]
    c = call["inputs"]
    keys = rec["param.keys"].clone().requires_grad_(True)
    values = rec["param.values"].clone().requires_grad_(True)
    q = c["q"].clone().requires_grad_(True)
    ref_v = c["ref_v"].clone().requires_grad_(True)
    gates = c["gates"].clone().requires_grad_(True) if "gates" in c else None
    out = ofw.forward_wo_past(q, ref_v, keys, values, cfg, rec["chunk_size"], gates, c.get("loss_mask"))
    assert torch.equal(out["indices"], call["indices"])
    for k in ("output", "scores", "losses", "addr_loss"):
        assert_rel_close(out[k], call[k], 1e-5, k)
    for a, e in zip(out["grad_norms"], call["grad_norms"]):
        assert_rel_close(a, e, 1e-5, "grad_norm")
    assert_rel_close(out["final"]["keys"], call["final.keys"], 1e-5, "final keys")
    assert_rel_close(out["final"]["values"], call["final.values"], 1e-5, "final values")
    out["output"].backward(c["dout"])
    assert_rel_close(q.grad, call["grad.q"], 1e-5, "dq")
    assert_rel_close(ref_v.grad, call["grad.ref_v"], 1e-5, "dref_v")
    assert_rel_close(keys.grad, call["grad.keys"], 1e-5, "dkeys")
    assert_rel_close(values.grad, call["grad.values"], 1e-5, "dvalues")
    if gates is not None:
        assert_rel_close(gates.grad, call["grad.gates"], 1e-5, "dgates")


def test_oracle_streaming_matches_reference():
    rec = load("stream")
    cfg = ofw.FwConfig.from_module_kwargs(rec["kwargs"])
    keys, values = rec["param.keys"].clone(), rec["param.values"].clone()
    past = (None,) * 6
    for n, call in enumerate(rec["calls"]):
        c = call["inputs"]
        with torch.no_grad():
            out = ofw.forward_w_past(c["q"], c["ref_v"], keys, values, cfg, rec["chunk_size"], c.get("gates"),
                                     c.get("loss_mask"), past, c["token_ids"])
        assert torch.equal(out["indices"], call["indices"]), n
        assert_rel_close(out["output"], call["output"], 1e-5, f"call {n} output")
        assert_rel_close(out["scores"], call["scores"], 1e-5, f"call {n} scores")
        assert (out["losses"] is None) == (call["losses"] is None)
        if call["losses"] is not None:
            assert_rel_close(out["losses"], call["losses"], 1e-5, f"call {n} losses")
        for a, e in zip(out["queues"], call["queues"]):
            assert (a is None) == (e is None)
            if e is not None:
                assert a.shape == e.shape
                assert_rel_close(a, e, 1e-5, f"call {n} queue")
        if out["final"] is not None:
            keys, values = out["final"]["keys"], out["final"]["values"]
        assert_rel_close(keys, call["final.keys"], 1e-5, f"call {n} keys")
        assert_rel_close(values, call["final.values"], 1e-5, f"call {n} values")
        past = out["queues"]
