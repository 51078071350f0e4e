"""Writes golden vectors of the reference's FastWeightProductKeyMemory
(fwpkm/fwpkm.py) on the CPU.

Run in a checkout that has the reference at REFERENCE (default
/root/reference):  python tests/golden/make_fwpkm_golden.py [case ...]
(all cases when none is named)

The reference module is imported only here, on the CPU (where its embedding
bag runs the index_select + sum forward, grad_wrapper:98-103, and the fp32
index_add_ first-order backward, legacy:147-167, under the same
EmbeddingBagBW double backward), to pin what no closed form covers: the
chunk loop of forward_wo_past (fwpkm.py:395-558) with the update between
chunks and the outer gradient through it, and the streaming queues of
forward_w_past (fwpkm.py:560-820) over successive calls.

Every parameter, input and upstream gradient is stored explicitly (float32),
with a SHA-256 of the inputs. Queries of the idw cases are scaled to 0.25 so
that query and key norms are alike and the distances spread. Inputs are drawn
(seed searched) so that every
top-k selection the reference makes has a relative gap of at least 1e-4
between the k-th and (k+1)-th score, per half and over the cartesian sums:
selections are then fixed by the scores, not by tie order.

Output: tests/golden/fwpkm_<case>.pt, a dict loadable with
torch.load(weights_only=True).
"""
from __future__ import annotations

import hashlib
import os
import sys
from pathlib import Path

import torch

REFERENCE = os.environ.get("REFERENCE", "/root/reference")
OUT = Path(__file__).resolve().parent
MIN_GAP = 1e-4

BASE = dict(mem_k_dim=32, mem_v_dim=16, mem_heads=2, mem_topk=8, mem_n_subkeys=64)
CASES = {
    # the fast-weight workload's choices (idw scores, lookahead 0, "me" address loss, lr 0.1), 2 chunks
    "idw_la0": dict(kw=dict(BASE, lookahead=0, qk_score_type="idw", learning_rate=0.1),
                    B=2, T=24, chunk=12, gates=False, mask=False, stream=False, q_scale=0.25),
    # dot scores, lookahead 1, gates and a loss mask, clipping, decay, temperature, 3 chunks (last short)
    "dot_la1": dict(kw=dict(BASE, lookahead=1, qk_score_type="dot_product", learning_rate=0.5, grad_clip=True,
                            weight_decay=0.01, score_temperature=0.5, addr_loss_weight=0.5),
                    B=2, T=26, chunk=12, gates=True, mask=True, stream=False, q_scale=1.0),
    # streaming: three calls of forward_w_past carrying the queues (7, 5, 6 tokens, chunk 8, lookahead 1)
    "stream": dict(kw=dict(BASE, lookahead=1, qk_score_type="idw", learning_rate=0.2),
                   B=2, T=[7, 5, 6], chunk=8, gates=True, mask=False, stream=True, q_scale=0.25),
}


def sha(*ts) -> str:
    h = hashlib.sha256()
    for t in ts:
        h.update(t.detach().contiguous().numpy().tobytes())
    return h.hexdigest()


def min_gap(s1, s2, k):
    """Smallest relative gap between the k-th and (k+1)-th score over both
    halves' sub-scores [N, H, n] and the cartesian sums of their top k+1."""
    gaps = []
    tops = []
    for s in (s1, s2):
        v = s.sort(dim=-1, descending=True).values
        gaps.append((v[..., k - 1] - v[..., k]).abs() / v[..., k - 1].abs().clamp_min(1e-6))
        tops.append(v[..., : k + 1])
    cand = (tops[0].unsqueeze(-1) + tops[1].unsqueeze(-2)).flatten(-2).sort(dim=-1, descending=True).values
    gaps.append((cand[..., k - 1] - cand[..., k]).abs() / cand[..., k - 1].abs().clamp_min(1e-6))
    return min(float(g.min()) for g in gaps)


def make(name, spec, Mem, seed):
    kw = spec["kw"]
    torch.manual_seed(0)
    mem = Mem(**kw)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        mem.keys.copy_((torch.rand(mem.keys.shape, generator=g) * 2 - 1) / kw["mem_k_dim"] ** 0.5)
        mem.values.copy_(torch.randn(mem.values.shape, generator=g) * kw["mem_v_dim"] ** -0.5)
    keys0, values0 = mem.keys.detach().clone(), mem.values.detach().clone()
    B, H, k_dim, v_dim = spec["B"], kw["mem_heads"], kw["mem_k_dim"], kw["mem_v_dim"]
    Ts = spec["T"] if spec["stream"] else [spec["T"]]
    calls = []
    for T in Ts:
        c = {"q": torch.randn((B, T, H * k_dim), generator=g) * spec["q_scale"],
             "ref_v": torch.randn((B, T, v_dim), generator=g)}
        if spec["gates"]:
            c["gates"] = torch.sigmoid(torch.randn((B, T), generator=g))
        if spec["mask"]:
            c["loss_mask"] = (torch.rand((B, T), generator=g) > 0.2).float()
        c["token_ids"] = torch.randint(0, 1000, (B, T), generator=g)
        c["dout"] = torch.randn((B, T, v_dim), generator=g)
        calls.append(c)

    # record every sub-score matrix the reference selects from
    seen = []
    orig = mem.get_indices

    def recording(query, keys):
        out = orig(query, keys)
        seen.append((out[4].detach().clone(), out[5].detach().clone()))
        return out

    mem.get_indices = recording
    mem.train()
    rec = {"kwargs": dict(kw), "chunk_size": spec["chunk"], "stream": spec["stream"], "seed": seed,
           "param.keys": keys0, "param.values": values0, "calls": []}
    past = (None,) * 6
    for c in calls:
        q = c["q"].clone().requires_grad_(True)
        ref_v = c["ref_v"].clone().requires_grad_(True)
        gates = c["gates"].clone().requires_grad_(True) if "gates" in c else None
        if spec["stream"]:
            out = mem(q=q, ref_v=ref_v, gates=gates, chunk_size=spec["chunk"], loss_mask=c.get("loss_mask"),
                      past_key_values=past, token_ids=c["token_ids"])
            past = out["past_key_values"]
            r = {"output": out["output"].detach().clone(), "indices": out["indices"].clone(),
                 "scores": out["scores"].detach().clone(),
                 "losses": out["losses"].clone() if out["losses"] is not None else None,
                 "addr_loss": out["addr_loss"].clone() if out["addr_loss"] is not None else None,
                 "queues": [t.detach().clone() if t is not None else None for t in past]}
        else:
            for p in mem.parameters():
                p.grad = None
            out = mem(q=q, ref_v=ref_v, gates=gates, chunk_size=spec["chunk"], loss_mask=c.get("loss_mask"),
                      past_key_values=None, token_ids=c["token_ids"])
            out["output"].backward(c["dout"])
            r = {"output": out["output"].detach().clone(), "indices": out["indices"].clone(),
                 "scores": out["scores"].detach().clone(), "losses": out["losses"].clone(),
                 "addr_loss": out["addr_loss"].clone(), "grad_norms": [t.clone() for t in out["grad_norms"]],
                 "grad.q": q.grad.clone(), "grad.ref_v": ref_v.grad.clone(),
                 "grad.keys": mem.keys.grad.clone(), "grad.values": mem.values.grad.clone()}
            if gates is not None:
                r["grad.gates"] = gates.grad.clone()
        r["final.keys"] = mem.keys.detach().clone()
        r["final.values"] = mem.values.detach().clone()
        r["inputs"] = {k: v.clone() for k, v in c.items()}
        r["sha256.inputs"] = sha(*[c[k] for k in sorted(c)])
        rec["calls"].append(r)
    gap = min(min_gap(s1, s2, kw["mem_topk"]) for s1, s2 in seen)
    return rec, gap


def main():
    sys.path.insert(0, REFERENCE)
    from fwpkm.fwpkm import FastWeightProductKeyMemory  # noqa: E402  (reference, CPU only)

    names = sys.argv[1:] or list(CASES)
    for name in names:
        for seed in range(100, 200):
            rec, gap = make(name, CASES[name], FastWeightProductKeyMemory, seed)
            if gap >= MIN_GAP:
                break
        else:
            raise RuntimeError(f"{name}: no seed with selection gaps >= {MIN_GAP}")
        rec["min_selection_gap"] = gap
        path = OUT / f"fwpkm_{name}.pt"
        torch.save(rec, path)
        print(f"wrote {path} ({path.stat().st_size} bytes, seed {rec['seed']}, min gap {gap:.2e})")


if __name__ == "__main__":
    main()
