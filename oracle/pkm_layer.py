"""PKM layer forward (HashingMemory): CPU restatement (test infrastructure only).

Functional form of pkm/memory.py:190-248 over an explicit parameter dict
(the reference's parameter names):
  X      = x.view(N, C)
  Q      = norm(X @ Wq^T + bq)                     QueryMLP (memory.py:333-349)
           norm: Qwen3RMSNorm (eps 1e-6)  or  BatchNorm1d in train mode (eps 1e-6)
  scores, idx = get_indices(Q.view(N*H, k), keys)  (memory.py:250-289, oracle.pkm)
  p      = softmax(scores.float(), -1).type_as(scores)   per head (memory.py:218)
  E      = embedding_bag(idx.view(N, H*knn), V, p.view(N, H*knn))   (memory.py:227)
  out    = value_proj(E * silu(swilu_projection(X)))   (memory.py:228-229)
Autograd through this function gives the reference's gradients (the top-k
selection is piecewise constant; scores reach keys and query through the
gathered sub-scores).
"""
from __future__ import annotations

from typing import Dict

import torch
import torch.nn.functional as F

from . import pkm as ref


def _norm(q: torch.Tensor, P: Dict[str, torch.Tensor], batchnorm: bool) -> torch.Tensor:
    if batchnorm:
        return F.batch_norm(q, None, None, P["query_proj.norm.weight"], P["query_proj.norm.bias"],
                            training=True, eps=1e-6)
    if "query_proj.norm.weight" in P:
        # Qwen3RMSNorm: float32 statistics, cast back, then the weight
        h = q.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)
        return P["query_proj.norm.weight"] * h.to(q.dtype)
    return q


def get_indices_differentiable(query: torch.Tensor, keys: torch.Tensor, heads: int, knn: int,
                               idx: torch.Tensor | None = None):
    """(scores, idx) [N*H, knn] with scores differentiable w.r.t. query and
    keys: the selection of oracle.pkm.get_indices (or a given one, [N*H, knn]),
    the values re-gathered from differentiable sub-scores (memory.py:267-285)."""
    N = query.shape[0] // heads
    if idx is None:
        with torch.no_grad():
            _, idx, _, _, _, _ = ref.get_indices(query.detach(), keys.detach(), heads, knn)
    idx = idx.reshape(N, heads, knn)
    k = query.shape[-1]
    half = k // 2
    q = query.reshape(N, heads, k)
    Kv = keys.reshape(heads, 2, -1, half)
    n = Kv.shape[2]
    s1 = torch.einsum("bhd,hnd->bhn", q[:, :, :half], Kv[:, 0])
    s2 = torch.einsum("bhd,hnd->bhn", q[:, :, half:], Kv[:, 1])
    scores = s1.gather(2, idx // n) + s2.gather(2, idx % n)
    return scores.reshape(N * heads, knn), idx.reshape(N * heads, knn)


def get_indices_torch(query: torch.Tensor, keys: torch.Tensor, heads: int, knn: int):
    """The reference's own op sequence (memory.py:250-289: einsum, topk,
    expand + add, topk, gather) in torch CPU ops; the CPU baseline's scoring.
    Equal to get_indices_differentiable on tie-free inputs."""
    N = query.shape[0] // heads
    k = query.shape[-1]
    half = k // 2
    q = query.view(N, heads, k)
    Kv = keys.view(heads, 2, -1, half)
    n = Kv.shape[2]
    s1 = torch.einsum("blh, lkh->blk", q[:, :, :half], Kv[:, 0])
    s2 = torch.einsum("blh, lkh->blk", q[:, :, half:], Kv[:, 1])
    s1, i1 = s1.topk(knn, dim=2, largest=True)
    s2, i2 = s2.topk(knn, dim=2, largest=True)
    cand = (s1.view(N, heads, knn, 1).expand(N, heads, knn, knn)
            + s2.view(N, heads, 1, knn).expand(N, heads, knn, knn)).view(N, heads, -1)
    cid = (i1.view(N, heads, knn, 1).expand(N, heads, knn, knn) * n
           + i2.view(N, heads, 1, knn).expand(N, heads, knn, knn)).view(N, heads, -1)
    scores, best = torch.topk(cand, k=knn, dim=2, largest=True, sorted=True)
    idx = cid.gather(2, best)
    return scores.view(N * heads, knn), idx.view(N * heads, knn)


def hashing_memory_forward(x: torch.Tensor, P: Dict[str, torch.Tensor], heads: int, knn: int,
                           batchnorm: bool = False, idx: torch.Tensor | None = None,
                           reference_ops: bool = False, bag_idx: torch.Tensor | None = None,
                           trace: dict | None = None):
    """(out [B, T, out_dim], indices [B, T, H*knn]) of HashingMemory.forward
    with swilu projection and no gating (the layer's defaults). `idx` forces
    the selection (to evaluate the layer at another implementation's ids);
    reference_ops selects with the reference's einsum/topk sequence instead of
    the stable-tie oracle (the CPU baseline). `bag_idx` [N*H, knn], when
    given, addresses P["values.weight"] instead of idx (a compact table of
    just the rows idx reads). `trace`, when given, receives the intermediate
    tensors (query Linear output "q_lin", swilu projection output "s", the
    value projection's input "h"), so a test can bound each output element by
    the sum of its terms' magnitudes."""
    B, T, C = x.shape
    X = x.reshape(-1, C)
    N = X.shape[0]
    q_lin = F.linear(X, P["query_proj.query_mlps.0.weight"], P.get("query_proj.query_mlps.0.bias"))
    q = _norm(q_lin, P, batchnorm)
    k_dim = q.shape[1] // heads
    if reference_ops:
        scores, idx = get_indices_torch(q.reshape(N * heads, k_dim), P["keys"], heads, knn)
    else:
        scores, idx = get_indices_differentiable(q.reshape(N * heads, k_dim), P["keys"], heads, knn, idx)
    p = F.softmax(scores.float(), dim=-1).type_as(scores)
    E = F.embedding_bag((idx if bag_idx is None else bag_idx).reshape(N, heads * knn), P["values.weight"],
                        per_sample_weights=p.reshape(N, heads * knn), mode="sum")
    s = F.linear(X, P["swilu_projection.weight"], P["swilu_projection.bias"])
    h = E * F.silu(s)
    out = F.linear(h, P["value_proj.weight"], P["value_proj.bias"])
    if trace is not None:
        trace.update(q_lin=q_lin, s=s, h=h)
    return out.reshape(B, T, -1), idx.reshape(B, T, -1)
