"""Writes golden vectors of the reference's FastWeightMLP (fwpkm/fwmlp.py) on
the CPU.

Run in a checkout that has the reference at REFERENCE (default
/root/reference):  python tests/golden/make_fwmlp_golden.py [case ...]
(all cases when none is named)

The reference module is imported only here, on the CPU, to pin what no closed
form covers: the chunk loop of forward_wo_past (fwmlp.py:192-318) with an SGD
step of every fast weight between chunks and the outer gradient through the
steps, and the streaming queues of forward_w_past (fwmlp.py:320-497) over
successive calls.

Every parameter, input and upstream gradient is stored explicitly (float32),
with a SHA-256 of the inputs. Output: tests/golden/fwmlp_<case>.pt, a dict
loadable with torch.load(weights_only=True).
"""
from __future__ import annotations

import hashlib
import os
import sys
from pathlib import Path

import torch

REFERENCE = os.environ.get("REFERENCE", "/root/reference")
OUT = Path(__file__).resolve().parent

BASE = dict(input_dim=12, output_dim=10, size=16)
CASES = {
    # lookahead 0, clipped steps, 3 chunks (the last one short)
    "la0": dict(kw=dict(BASE, lookahead=0, learning_rate=0.5, grad_clip=True),
                B=2, T=[20], chunk=8, mask=False, stream=False),
    # lookahead 2 "mean" targets, mae loss, weight decay, unclipped steps, a loss mask
    "la2_mean": dict(kw=dict(BASE, lookahead=2, lookahead_strategy="mean", loss_type="mae", weight_decay=0.01,
                             learning_rate=0.3, grad_clip=False),
                     B=2, T=[22], chunk=8, mask=True, stream=False),
    # lookahead 1 "last" targets
    "la1_last": dict(kw=dict(BASE, lookahead=1, lookahead_strategy="last", learning_rate=0.2),
                     B=3, T=[17], chunk=6, mask=False, stream=False),
    # streaming: three calls of forward_w_past carrying the queues (7, 5, 6 tokens, chunk 4, lookahead 1)
    "stream": dict(kw=dict(BASE, lookahead=1, learning_rate=0.2),
                   B=2, T=[7, 5, 6], chunk=4, mask=True, stream=True),
}


def sha(*ts) -> str:
    h = hashlib.sha256()
    for t in ts:
        h.update(t.detach().contiguous().numpy().tobytes())
    return h.hexdigest()


def make(spec, Mlp, seed):
    kw = spec["kw"]
    torch.manual_seed(seed)
    mlp = Mlp(**kw)
    mlp.reset_parameters()
    # biases away from zero, so that their steps and gradients are exercised from the first chunk
    with torch.no_grad():
        for n, p in mlp.named_parameters():
            if n.startswith("b_"):
                p.normal_(0.0, 0.1)
    params0 = {n: p.detach().clone() for n, p in mlp.named_parameters()}
    g = torch.Generator().manual_seed(seed + 1)
    calls = []
    for T in spec["T"]:
        c = {"q": torch.randn(spec["B"], T, kw["input_dim"], generator=g),
             "ref_v": torch.randn(spec["B"], T, kw["output_dim"], generator=g),
             "dout": torch.randn(spec["B"], T, kw["output_dim"], generator=g)}
        if spec["mask"]:
            c["loss_mask"] = (torch.rand(spec["B"], T, generator=g) > 0.25).float()
        calls.append(c)
    mlp.train()
    rec = {"kwargs": dict(kw), "chunk_size": spec["chunk"], "stream": spec["stream"], "seed": seed,
           "params0": params0, "calls": []}
    past = (None,) * 6
    for c in calls:
        q = c["q"].clone().requires_grad_(True)
        ref_v = c["ref_v"].clone().requires_grad_(True)
        if spec["stream"]:
            out = mlp(q=q, ref_v=ref_v, chunk_size=spec["chunk"], loss_mask=c.get("loss_mask"), past_key_values=past)
            past = out["past_key_values"]
            r = {"output": out["output"].detach().clone(),
                 "losses": out["losses"].clone() if out["losses"] is not None else None,
                 "grad_norms": [t.clone() for t in out["grad_norms"]] if out["grad_norms"] is not None else None,
                 "queues": [t.detach().clone() if t is not None else None for t in past]}
        else:
            for p in mlp.parameters():
                p.grad = None
            out = mlp(q=q, ref_v=ref_v, chunk_size=spec["chunk"], loss_mask=c.get("loss_mask"))
            out["output"].backward(c["dout"])
            r = {"output": out["output"].detach().clone(), "losses": out["losses"].clone(),
                 "grad_norms": [t.clone() for t in out["grad_norms"]],
                 "grad.q": q.grad.clone(), "grad.ref_v": ref_v.grad.clone(),
                 "grad.params": {n: p.grad.clone() for n, p in mlp.named_parameters()}}
        r["final.params"] = {n: p.detach().clone() for n, p in mlp.named_parameters()}
        r["inputs"] = {k: v.clone() for k, v in c.items()}
        r["sha256.inputs"] = sha(*[c[k] for k in sorted(c)])
        rec["calls"].append(r)
    return rec


def main():
    sys.path.insert(0, REFERENCE)
    from fwpkm.fwmlp import FastWeightMLP  # noqa: E402  (reference, CPU only)

    names = sys.argv[1:] or list(CASES)
    for i, name in enumerate(names):
        rec = make(CASES[name], FastWeightMLP, 300 + i)
        path = OUT / f"fwmlp_{name}.pt"
        torch.save(rec, path)
        print(f"wrote {path} ({path.stat().st_size} bytes, seed {rec['seed']})")


if __name__ == "__main__":
    main()
