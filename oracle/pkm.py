"""Product-key retrieval: CPU restatement (test infrastructure only).

Semantics (reference HashingMemory.get_indices, pkm/memory.py:250-289, and
FastWeightProductKeyMemory.get_indices / compute_qk_scores,
fwpkm/fwpkm.py:853-934):
  query [N, H, k] split into halves q_0 = q[..., :k/2], q_1 = q[..., k/2:]
  keys [2*H*n, k/2] viewed (H, 2, n, k/2): key (h, c, i) is row (2h + c) * n + i
  s_c = score(q_c, K_c)                    rounded to the module dtype
        dot: einsum("blh,lkh->blk")       (memory.py:267-268, fwpkm.py:860-861)
        idw: -log(1e-3 + cdist(q, k)^2)   (fwpkm.py:862-866)
  (v_c, i_c) = topk(s_c, knn), sorted best first (memory.py:270-271)
  cand[a * knn + b] = v_0[a] + v_1[b]      rounded to the dtype (memory.py:274-277)
  cid[a * knn + b]  = i_0[a] * n + i_1[b]  (memory.py:278-281)
  (scores, best) = topk(cand, knn, sorted); idx = cid.gather(best)  (memory.py:284-285)

torch.topk leaves the order of equal values unspecified; this restatement
(and the HIP kernel) orders equal values by the smaller position: sub-key
index for the per-half top-k, flat position a * knn + b for the cartesian one.
"""
from __future__ import annotations

from typing import Tuple

import torch

DOT, IDW = "dot", "idw"


def key_rows(H: int, n: int, c: int, h: int, i):
    """Row of key (h, c, i) in the [2*H*n, half] table (keys.view(H, 2, n, half),
    pkm/memory.py:257-260, fwpkm/fwpkm.py:891-893)."""
    return (2 * h + c) * n + i


def sub_scores(query: torch.Tensor, keys: torch.Tensor, heads: int, score_type: str = DOT,
               out_dtype: torch.dtype | None = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sub-key scores s_0, s_1 [N, H, n], computed in float64 from the stored
    inputs and rounded once to out_dtype (default: the input dtype).
    Reference: memory.py:262-268 (dot), fwpkm.py:853-869 (dot / idw)."""
    k = query.shape[-1]
    N = query.numel() // (heads * k)  # query [N, H, k] or [N * H, k]
    half = k // 2
    q = query.reshape(N, heads, k).to(torch.float64)
    K = keys.to(torch.float64).reshape(heads, 2, -1, half)
    out = []
    for c in range(2):
        qc = q[:, :, c * half:(c + 1) * half]  # [N, H, half]
        Kc = K[:, c]  # [H, n, half]
        dot = torch.einsum("bhd,hnd->bhn", qc, Kc)
        if score_type == DOT:
            s = dot
        elif score_type == IDW:
            d2 = (qc * qc).sum(-1)[:, :, None] + (Kc * Kc).sum(-1)[None, :, :] - 2.0 * dot
            s = -torch.log(1e-3 + d2.clamp_min(0.0))
        else:
            raise ValueError(score_type)
        out.append(s.to(out_dtype or query.dtype))
    return out[0], out[1]


def topk_stable(x: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k along the last dim, best first; equal values in index order
    (torch.topk with a fixed tie order, memory.py:270-271)."""
    v, i = torch.sort(x, dim=-1, descending=True, stable=True)
    return v[..., :k], i[..., :k]


def _round_sum(x64: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Sum of two values of `dtype` computed in float64, rounded as the
    reference's `dtype + dtype` is: float32 arithmetic, then `dtype`.
    (A float64 sum of two floats of <= 24 bits, rounded once to float32, is
    the correctly rounded float32 sum: 53 >= 2 * 24 + 2.)"""
    if dtype == torch.float64:
        return x64
    return x64.to(torch.float32).to(dtype)


def select(s1: torch.Tensor, s2: torch.Tensor, knn: int):
    """Per-half top-k and the full knn x knn cartesian top-k from given
    sub-scores [N, H, n] (memory.py:270-289, fwpkm.py:904-921).
    Returns scores [N, H, knn] (s dtype), idx, i1, i2 [N, H, knn] int64."""
    n = s1.shape[-1]
    v1, i1 = topk_stable(s1, knn)
    v2, i2 = topk_stable(s2, knn)
    N, H = s1.shape[:2]
    cand = _round_sum(v1[..., :, None].to(torch.float64) + v2[..., None, :].to(torch.float64), s1.dtype)
    cand = cand.reshape(N, H, knn * knn)
    cid = (i1[..., :, None] * n + i2[..., None, :]).reshape(N, H, knn * knn)
    scores, best = topk_stable(cand, knn)
    idx = cid.gather(2, best)
    return scores, idx, i1, i2


def get_indices(query: torch.Tensor, keys: torch.Tensor, heads: int, knn: int, score_type: str = DOT):
    """FastWeightProductKeyMemory.get_indices 6-tuple (fwpkm.py:871-934):
    scores, idx, i1, i2 [N, H, knn]; s1, s2 [N, H, n]. HashingMemory.get_indices
    (memory.py:250-289) returns scores, idx viewed [N*H, knn]."""
    s1, s2 = sub_scores(query, keys, heads, score_type)
    scores, idx, i1, i2 = select(s1, s2, knn)
    return scores, idx, i1, i2, s1, s2


def select_pruned(s1: torch.Tensor, s2: torch.Tensor, knn: int):
    """Cartesian top-k over the pairs (a, b) with (a+1)(b+1) <= knn only: the
    HIP kernel's candidate set. Every other pair is preceded, in (value desc,
    a*knn+b asc) order, by the >= knn pairs (a', b') <= (a, b), so the result
    equals select()'s, ties included. Kept here to check that claim."""
    n = s1.shape[-1]
    v1, i1 = topk_stable(s1, knn)
    v2, i2 = topk_stable(s2, knn)
    pairs = [(a, b) for a in range(knn) for b in range(knn) if (a + 1) * (b + 1) <= knn]
    A = torch.tensor([p[0] for p in pairs])
    Bc = torch.tensor([p[1] for p in pairs])
    cand = _round_sum(v1[..., A].to(torch.float64) + v2[..., Bc].to(torch.float64), s1.dtype)
    scores, best = topk_stable(cand, knn)  # pairs are in increasing a*knn+b order
    idx = (i1[..., A] * n + i2[..., Bc]).gather(2, best)
    return scores, idx, i1, i2


def brute_force_topk_pairs(s1: torch.Tensor, s2: torch.Tensor, knn: int):
    """Exact top-knn over all n*n pair sums of one (token, head) in Python
    (tiny n only): returns [(value, i1 * n + i2)] best first, ties by the
    smaller flat id."""
    n = s1.shape[-1]
    vals = []
    for i in range(n):
        for j in range(n):
            v = _round_sum(torch.tensor(float(s1[i]) + float(s2[j]), dtype=torch.float64), s1.dtype)
            vals.append((float(v), i * n + j))
    vals.sort(key=lambda t: (-t[0], t[1]))
    return vals[:knn]


def score_grad_dense(idx: torch.Tensor, d: torch.Tensor, n: int, d_s1: torch.Tensor | None = None,
                     d_s2: torch.Tensor | None = None) -> torch.Tensor:
    """Gradient of the full sub-score matrices [H, 2, N, n] from the gradient d
    [N, H, knn] of scores = s1[id // n] + s2[id % n] (memory.py:274-285 with
    the selection fixed), plus optional dense gradients of s1, s2 [N, H, n]:
    float32 sums in j order, then the dense term, rounded once to d's dtype."""
    N, H, knn = idx.shape
    out = torch.zeros((H, 2, N, n), dtype=torch.float32)
    i1, i2 = idx // n, idx % n
    df = d.float()
    for j in range(knn):  # j order, as the reference's index accumulation of a row
        for c, ic in ((0, i1), (1, i2)):
            view = out[:, c]  # [H, N, n]
            view.scatter_add_(2, ic[:, :, j].t().reshape(H, N, 1), df[:, :, j].t().reshape(H, N, 1))
    if d_s1 is not None:
        out[:, 0] += d_s1.float().permute(1, 0, 2)
    if d_s2 is not None:
        out[:, 1] += d_s2.float().permute(1, 0, 2)
    return out.to(d.dtype)
