"""Weighted embedding bag: CPU restatement (test infrastructure only).

Semantics (reference):
  forward   out[b] = sum_j w[b,j] * W[idx[b,j]], float32 accumulation in j
            order, one rounding to W's dtype
            (pkm/xformer_embeddingbag.py:97-113, output dtype :123)
  backward  gW[r] = sum_{idx[b,j]==r} w[b,j] * g[b]   float32, dense, W dtype
            gw[b,j] = <W[idx[b,j]], g[b]>              float32 dot, w dtype
            (pkm/xformer_embeddingbag.py:291-328; fwpkm/xformer_embeddingbag_legacy.py:160-167)
  double    d_g[b] = sum_j a[b,j] * gbar[idx[b,j]];  d_a[b,j] = <gbar[idx[b,j]], g[b]>
            (fwpkm/xformer_embeddingbag_grad_wrapper.py:55-74)

Indices outside [0, K) contribute nothing and get a zero weight gradient (the
documented behaviour of the HIP library; the reference leaves them undefined).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def _valid_mask(indices: torch.Tensor, K: int) -> torch.Tensor:
    return (indices >= 0) & (indices < K)


def eb_forward(indices: torch.Tensor, weight: torch.Tensor, psw: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Reference embedding_bag_k (pkm/xformer_embeddingbag.py:106-113)."""
    B, L = indices.shape
    K, D = weight.shape
    acc_dtype = torch.float64 if weight.dtype == torch.float64 else torch.float32
    acc = torch.zeros((B, D), dtype=acc_dtype)
    valid = _valid_mask(indices, K)
    safe = torch.where(valid, indices, torch.zeros_like(indices))
    for j in range(L):  # :108, j in increasing order
        rows = weight[safe[:, j]].to(acc_dtype)  # :111
        w = psw[:, j].to(acc_dtype) if psw is not None else torch.ones(B, dtype=acc_dtype)  # :110
        w = torch.where(valid[:, j], w, torch.zeros_like(w))
        acc = acc + rows * w[:, None]  # :112
    return acc.to(weight.dtype)  # :113 store into weight.dtype (:123)


def eb_forward_library(indices: torch.Tensor, weight: torch.Tensor, psw: Optional[torch.Tensor]) -> torch.Tensor:
    """The reference's CPU path: F.embedding_bag (pkm/xformer_embeddingbag.py:436-437)."""
    return F.embedding_bag(indices, weight, per_sample_weights=psw, mode="sum")


def eb_backward(
    indices: torch.Tensor, weight: torch.Tensor, psw: Optional[torch.Tensor], grad: torch.Tensor
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Reference aggregate_gradient_for_embedding_k (pkm/xformer_embeddingbag.py:312-328) and
    _embedding_bag_bw_native (fwpkm/xformer_embeddingbag_legacy.py:160-167).

    gW rows are summed in increasing flat position b*L+j (index_add_ walks the
    flattened index in order)."""
    B, L = indices.shape
    K, D = weight.shape
    acc_dtype = torch.float64 if weight.dtype == torch.float64 else torch.float32
    valid = _valid_mask(indices, K).reshape(-1)
    flat = indices.reshape(-1)
    g = grad.to(acc_dtype)
    w = psw.to(acc_dtype) if psw is not None else torch.ones((B, L), dtype=acc_dtype)
    contrib = (g[:, None, :] * w[:, :, None]).reshape(B * L, D)  # legacy:163
    gW = torch.zeros((K, D), dtype=acc_dtype)
    gW.index_add_(0, flat[valid], contrib[valid])  # legacy:164-165
    gpsw = None
    if psw is not None:
        safe = torch.where(valid, flat, torch.zeros_like(flat))
        rows = weight[safe].to(acc_dtype).view(B, L, D)
        gpsw = (rows * g[:, None, :]).sum(-1)  # legacy:162; xformer_embeddingbag.py:325-326
        gpsw = torch.where(valid.view(B, L), gpsw, torch.zeros_like(gpsw)).to(psw.dtype)
    return gW.to(weight.dtype), gpsw


def eb_double_backward(
    indices: torch.Tensor, a: Optional[torch.Tensor], grad: torch.Tensor, gbar: torch.Tensor
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Reference EmbeddingBagBW.backward (fwpkm/xformer_embeddingbag_grad_wrapper.py:55-74)."""
    B, L = indices.shape
    K, D = gbar.shape
    acc_dtype = torch.float64 if gbar.dtype == torch.float64 else torch.float32
    valid = _valid_mask(indices, K)
    safe = torch.where(valid, indices, torch.zeros_like(indices))
    gathered = gbar[safe.reshape(-1)].to(acc_dtype).view(B, L, D)  # :60
    gathered = gathered * valid[:, :, None].to(acc_dtype)
    if a is not None:
        d_g = (a.to(acc_dtype)[:, :, None] * gathered).sum(1)  # :66
        d_a = (gathered * grad.to(acc_dtype)[:, None, :]).sum(-1)  # :68
        return d_g.to(grad.dtype), d_a.to(a.dtype)
    return gathered.sum(1).to(grad.dtype), None  # :70


def brute_force_forward(indices, weight, psw):
    """Pure-Python loops (tiny inputs only), float64."""
    B, L = indices.shape
    K, D = weight.shape
    out = [[0.0] * D for _ in range(B)]
    for b in range(B):
        for j in range(L):
            r = int(indices[b, j])
            if not 0 <= r < K:
                continue
            w = 1.0 if psw is None else float(psw[b, j])
            for d in range(D):
                out[b][d] += w * float(weight[r, d])
    return torch.tensor(out, dtype=torch.float64)


def brute_force_backward(indices, weight, psw, grad):
    B, L = indices.shape
    K, D = weight.shape
    gW = [[0.0] * D for _ in range(K)]
    gp = [[0.0] * L for _ in range(B)]
    for b in range(B):
        for j in range(L):
            r = int(indices[b, j])
            if not 0 <= r < K:
                continue
            w = 1.0 if psw is None else float(psw[b, j])
            for d in range(D):
                gW[r][d] += w * float(grad[b, d])
                gp[b][j] += float(weight[r, d]) * float(grad[b, d])
    return torch.tensor(gW, dtype=torch.float64), torch.tensor(gp, dtype=torch.float64)


def brute_force_double_backward(indices, a, grad, gbar):
    B, L = indices.shape
    K, D = gbar.shape
    dg = [[0.0] * D for _ in range(B)]
    da = [[0.0] * L for _ in range(B)]
    for b in range(B):
        for j in range(L):
            r = int(indices[b, j])
            if not 0 <= r < K:
                continue
            w = 1.0 if a is None else float(a[b, j])
            for d in range(D):
                dg[b][d] += w * float(gbar[r, d])
                da[b][j] += float(gbar[r, d]) * float(grad[b, d])
    return torch.tensor(dg, dtype=torch.float64), torch.tensor(da, dtype=torch.float64)
