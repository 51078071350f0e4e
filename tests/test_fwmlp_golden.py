"""FastWeightMLP (modelos_amd/fwpkm/fwmlp.py) against the reference's own
outputs, on the CPU.

tests/golden/fwmlp_*.pt were written by the reference's FastWeightMLP
(fwpkm/fwmlp.py:20-522) by tests/golden/make_fwmlp_golden.py: explicit
parameters, inputs, upstream gradients and loss masks, and the reference's
outputs, per-example losses, grad norms, final (stored) fast weights, and for
the chunked cases the outer gradients of the queries, the targets and every
parameter through the in-context SGD steps; for the streaming case three
successive forward_w_past calls with the queues they carry.
"""
from pathlib import Path

import pytest
import torch

from modelos_amd.fwpkm.fwmlp import FastWeightMLP

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ["la0", "la2_mean", "la1_last", "stream"]
TOL = dict(rtol=1e-5, atol=1e-5)


def load(case):
    return torch.load(GOLDEN / f"fwmlp_{case}.pt", weights_only=True)


def build(rec):
    mlp = FastWeightMLP(**rec["kwargs"])
    with torch.no_grad():
        for n, p in mlp.named_parameters():
            p.copy_(rec["params0"][n])
    mlp.train()
    return mlp


def close(a, b, what):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    torch.testing.assert_close(a, b, **TOL, msg=lambda m: f"{what}: {m}")


@pytest.mark.parametrize("case", [c for c in CASES if c != "stream"])
def test_chunked_fit_and_outer_gradients(case):
    rec = load(case)
    mlp = build(rec)
    for call in rec["calls"]:
        inp = call["inputs"]
        q = inp["q"].clone().requires_grad_(True)
        ref_v = inp["ref_v"].clone().requires_grad_(True)
        out = mlp(q=q, ref_v=ref_v, chunk_size=rec["chunk_size"], loss_mask=inp.get("loss_mask"))
        out["output"].backward(inp["dout"])
        close(out["output"].detach(), call["output"], "output")
        close(out["losses"], call["losses"], "losses")
        assert len(out["grad_norms"]) == len(call["grad_norms"])
        for i, (a, b) in enumerate(zip(out["grad_norms"], call["grad_norms"])):
            close(a, b, f"grad_norms[{i}]")
        close(q.grad, call["grad.q"], "grad.q")
        close(ref_v.grad, call["grad.ref_v"], "grad.ref_v")
        for n, p in mlp.named_parameters():
            close(p.grad, call["grad.params"][n], f"grad.{n}")
            close(p.detach(), call["final.params"][n], f"final.{n}")
        assert out["past_key_values"] is None


def test_streaming_queues():
    rec = load("stream")
    mlp = build(rec)
    past = (None,) * 6
    for k, call in enumerate(rec["calls"]):
        inp = call["inputs"]
        out = mlp(q=inp["q"], ref_v=inp["ref_v"], chunk_size=rec["chunk_size"], loss_mask=inp.get("loss_mask"),
                  past_key_values=past)
        past = out["past_key_values"]
        close(out["output"].detach(), call["output"], f"call {k} output")
        if call["losses"] is None:
            assert out["losses"] is None
        else:
            close(out["losses"], call["losses"], f"call {k} losses")
        if call["grad_norms"] is None:
            assert out["grad_norms"] is None
        else:
            for i, (a, b) in enumerate(zip(out["grad_norms"], call["grad_norms"])):
                close(a, b, f"call {k} grad_norms[{i}]")
        assert len(past) == len(call["queues"])
        for i, (a, b) in enumerate(zip(past, call["queues"])):
            if b is None:
                assert a is None, f"call {k} queue {i}"
            else:
                close(a.detach(), b, f"call {k} queue {i}")
        for n, p in mlp.named_parameters():
            close(p.detach(), call["final.params"][n], f"call {k} final.{n}")
