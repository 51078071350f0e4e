"""Host side of product-key retrieval: scores + per-half top-k + cartesian top-k.

`score_topk` runs the fused HIP kernel (pkm_score_topk) on torch's current
stream. `product_key_topk` wraps it in autograd:

  * the returned top-knn scores are differentiable w.r.t. query and keys;
    their gradient is sparse (each score touches one key row per half) and is
    computed with the embedding-bag kernels on the key table:
      dq[t,h,c]  = sum_j dscore[t,h,j] * d s_c / d q      (an embedding-bag forward)
      dkeys[row] = sum_{(t,h,j) -> row} dscore * d s / d k (an embedding-bag backward)
  * the optional full sub-score matrices s_1, s_2 (fast-weight PKM) are
    differentiable too; their dense gradient goes through batched GEMMs.

Reference: HashingMemory.get_indices (pkm/memory.py:250-289),
FastWeightProductKeyMemory.compute_qk_scores / get_indices
(fwpkm/fwpkm.py:853-934); autograd of einsum/cdist -> topk -> expand+add ->
topk -> gather there gives the same gradients.

There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib
from .embedding_bag import _aligned, _require_device, eb_backward, eb_forward

SCORE_TYPES = ("dot", "idw")


def _check(query: torch.Tensor, keys: torch.Tensor, heads: int, knn: int, score_type: str):
    if score_type not in SCORE_TYPES:
        raise ValueError(f"score_type must be one of {SCORE_TYPES}, got {score_type!r}")
    if keys.dim() != 2:
        raise ValueError(f"keys must be [2 * heads * n_keys, k_dim // 2], got shape {tuple(keys.shape)}")
    half = keys.shape[1]
    k_dim = 2 * half
    if query.shape[-1] != k_dim:
        raise ValueError(f"query last dim {query.shape[-1]} != 2 * keys.shape[1] = {k_dim}")
    if query.numel() % (heads * k_dim) != 0:
        raise ValueError(f"query of shape {tuple(query.shape)} is not [tokens, {heads}, {k_dim}]")
    if keys.shape[0] % (2 * heads) != 0:
        raise ValueError(f"keys rows {keys.shape[0]} not a multiple of 2 * heads = {2 * heads}")
    if query.dtype != keys.dtype:
        raise TypeError(f"query dtype {query.dtype} != keys dtype {keys.dtype}")
    n = keys.shape[0] // (2 * heads)
    if not 1 <= knn <= n:
        raise ValueError(f"knn must be in [1, n_keys={n}], got {knn}")
    return query.numel() // (heads * k_dim), n, half


def score_topk(
    query: torch.Tensor,
    keys: torch.Tensor,
    heads: int,
    knn: int,
    score_type: str = "dot",
    sub_outputs: bool = False,
):
    """Forward only (no autograd).

    query: [tokens, heads, k_dim] (or any view with that many elements, e.g.
    [tokens * heads, k_dim]); keys: [2 * heads * n_keys, k_dim // 2].
    Returns scores, indices [tokens * heads, knn] and, with sub_outputs,
    additionally i1, i2 [tokens, heads, knn] and s1, s2 [tokens, heads, n_keys].
    """
    N, n, half = _check(query, keys, heads, knn, score_type)
    dev = _require_device(query, keys)
    query = _aligned(query)
    keys = _aligned(keys)
    dt = query.dtype
    scores = torch.empty((N * heads, knn), dtype=dt, device=dev)
    indices = torch.empty((N * heads, knn), dtype=torch.long, device=dev)
    i1 = i2 = s1 = s2 = None
    if sub_outputs:
        i1 = torch.empty((N, heads, knn), dtype=torch.long, device=dev)
        i2 = torch.empty((N, heads, knn), dtype=torch.long, device=dev)
        s1 = torch.empty((N, heads, n), dtype=dt, device=dev)
        s2 = torch.empty((N, heads, n), dtype=dt, device=dev)
    _lib.call(
        "pkm_score_topk",
        _lib.ptr(query), _lib.ptr(keys), N, heads, n, half, knn,
        _lib.SCORE_CODES[score_type], _lib.dtype_code(query),
        _lib.ptr(scores), _lib.ptr(indices), _lib.ptr(i1), _lib.ptr(i2), _lib.ptr(s1), _lib.ptr(s2),
        _lib.stream_of(dev),
    )
    if sub_outputs:
        return scores, indices, i1, i2, s1, s2
    return scores, indices


def _key_rows(indices: torch.Tensor, heads: int, n: int) -> torch.Tensor:
    """Key-table rows of the two halves of every selected slot:
    [tokens * heads * 2, knn], bag (t, h, c) = (t * heads + h) * 2 + c, row
    (2h + c) * n + i_c with i_0 = id // n, i_1 = id % n (memory.py:278-281)."""
    NH, knn = indices.shape
    h = (torch.arange(NH, device=indices.device) % heads)[:, None]
    r0 = (2 * h) * n + torch.div(indices, n, rounding_mode="floor")
    r1 = (2 * h + 1) * n + torch.remainder(indices, n)
    return torch.stack((r0, r1), dim=1).reshape(NH * 2, knn)


def _sparse_grads(query, keys, indices, d_scores, heads, n, score_type):
    """Gradient of the selected top-knn scores w.r.t. query ([N*H*2, half]
    float32) and keys ([2Hn, half] float32)."""
    NH, knn = indices.shape
    half = keys.shape[1]
    rows = _key_rows(indices, heads, n)
    q2 = query.reshape(NH * 2, half)
    w = d_scores.float()[:, None, :].expand(NH, 2, knn).reshape(NH * 2, knn)
    if score_type == "dot":
        # s = <q, k>: dq = sum_j w_j k_j, dk_r = sum_{j -> r} w_j q_j
        dq = eb_forward(rows, keys, w).float()
        dk, _ = eb_backward(rows, keys, w, q2)
        return dq, dk.float()
    # s = -log(1e-3 + max(d2, 0)), d2 = |q - k|^2:
    #   ds/dq = 2 u (k - q), ds/dk = 2 u (q - k), u = 1 / (1e-3 + d2) (0 where d2 < 0)
    keys32, q32 = keys.float(), q2.float()
    _, dots = eb_backward(rows, keys32, torch.zeros_like(w), q32)  # <k_row, q> per slot
    qn = (q32 * q32).sum(-1)
    kn = (keys32 * keys32).sum(-1)
    d2 = qn[:, None] + kn[rows] - 2.0 * dots
    u = torch.where(d2 >= 0, w / (1e-3 + d2.clamp_min(0.0)), torch.zeros_like(d2))
    dq = 2.0 * eb_forward(rows, keys32, u) - 2.0 * q32 * u.sum(-1, keepdim=True)
    gk, _ = eb_backward(rows, keys32, u, q32)
    usum = torch.zeros(keys.shape[0], dtype=torch.float32, device=keys.device)
    usum.index_add_(0, rows.reshape(-1), u.reshape(-1))
    dk = 2.0 * gk - 2.0 * keys32 * usum[:, None]
    return dq, dk


def _dense_grads(query, keys, d_s, heads, n, score_type, dq, dk):
    """Adds the gradient of the full sub-score matrices s_c [N, H, n] (float32,
    batched GEMMs per head) to dq [N, H, 2, half] and dk [H, 2, n, half]."""
    half = keys.shape[1]
    N = query.numel() // (heads * 2 * half)
    q = query.reshape(N, heads, 2, half).float()
    K = keys.reshape(heads, 2, n, half).float()
    for c, g in enumerate(d_s):
        if g is None:
            continue
        G = g.float().permute(1, 0, 2).contiguous()  # [H, N, n]
        qc = q[:, :, c].permute(1, 0, 2).contiguous()  # [H, N, half]
        Kc = K[:, c].contiguous()  # [H, n, half]
        if score_type == "idw":
            dots = torch.bmm(qc, Kc.transpose(1, 2).contiguous())  # [H, N, n]
            d2 = (qc * qc).sum(-1)[:, :, None] + (Kc * Kc).sum(-1)[:, None, :] - 2.0 * dots
            U = torch.where(d2 >= 0, G / (1e-3 + d2.clamp_min(0.0)), torch.zeros_like(d2))
            gq = 2.0 * (torch.bmm(U, Kc) - qc * U.sum(-1, keepdim=True))
            gk = 2.0 * (torch.bmm(U.transpose(1, 2).contiguous(), qc) - Kc * U.sum(1)[:, :, None])
        else:
            gq = torch.bmm(G, Kc)
            gk = torch.bmm(G.transpose(1, 2).contiguous(), qc)
        dq[:, :, c] += gq.permute(1, 0, 2)
        dk[:, c] += gk


class ProductKeyTopK(torch.autograd.Function):
    """Differentiable product-key retrieval (scores w.r.t. query and keys)."""

    @staticmethod
    def forward(ctx, query, keys, heads, knn, score_type, sub_outputs):
        outs = score_topk(query, keys, heads, knn, score_type, sub_outputs)
        ctx.heads, ctx.knn, ctx.score_type, ctx.sub_outputs = heads, knn, score_type, sub_outputs
        ctx.n = keys.shape[0] // (2 * heads)
        ctx.query_shape = query.shape
        ctx.save_for_backward(query, keys, outs[1])
        ctx.mark_non_differentiable(*(outs[1:4] if sub_outputs else outs[1:2]))
        return outs

    @staticmethod
    def backward(ctx, d_scores, d_indices, *rest):
        query, keys, indices = ctx.saved_tensors
        heads, n = ctx.heads, ctx.n
        half = keys.shape[1]
        NH = indices.shape[0]
        N = NH // heads
        qc = _aligned(query)
        kc = _aligned(keys)
        dq = torch.zeros((N, heads, 2, half), dtype=torch.float32, device=query.device)
        dk = torch.zeros((heads, 2, n, half), dtype=torch.float32, device=keys.device)
        if d_scores is not None and NH > 0:
            sq, sk = _sparse_grads(qc, kc, indices, d_scores.contiguous(), heads, n, ctx.score_type)
            dq += sq.reshape(N, heads, 2, half)
            dk += sk.reshape(heads, 2, n, half)
        if ctx.sub_outputs and N > 0:
            d_s = (rest[2], rest[3])
            if any(g is not None for g in d_s):
                _dense_grads(qc, kc, d_s, heads, n, ctx.score_type, dq, dk)
        d_query = dq.to(query.dtype).reshape(ctx.query_shape) if ctx.needs_input_grad[0] else None
        d_keys = dk.to(keys.dtype).reshape(keys.shape) if ctx.needs_input_grad[1] else None
        return d_query, d_keys, None, None, None, None


def product_key_topk(
    query: torch.Tensor,
    keys: torch.Tensor,
    heads: int,
    knn: int,
    score_type: str = "dot",
    sub_outputs: bool = False,
) -> Tuple[torch.Tensor, ...]:
    """Autograd version of score_topk (same arguments and outputs)."""
    return ProductKeyTopK.apply(query, keys, heads, knn, score_type, sub_outputs)


def sparse_key_rows(indices: torch.Tensor, heads: int, n_keys: int) -> torch.Tensor:
    """Public form of the key-row mapping used by the backward (for tests)."""
    return _key_rows(indices, heads, n_keys)


__all__ = ["score_topk", "product_key_topk", "ProductKeyTopK", "sparse_key_rows", "SCORE_TYPES"]
