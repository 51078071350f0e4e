"""Marginal-entropy address loss of the fast-weight memory on the HIP kernels
(pkm_me_grad_fwd / pkm_me_grad_hvp): the loss value and the key table's
gradient in one pass, differentiable in turn (the outer backward through an
inner update step).

Reference: compute_marginal_entropy / compute_addr_loss
(fwpkm/fwpkm.py:117-147, 233-264) and the keys' gradient update_fw takes of
them with torch.autograd.grad(..., create_graph=True) (fwpkm/fwpkm.py:274-367).

The kernels take every (token, key) entry of the sub-score rows, lane-parallel
(a row's mask is its topk best entries and every entry tied with the last of
them: a few more than topk for float32 scores, most of the row for 16-bit idw
scores, which tie heavily); the products with the queries, the keys and the
outer gradient are batched GEMMs over dense [2 heads, tokens, n] operands. The
double backward is split along the reference's graph: the part through the
sub-scores comes back as their gradient, which the retrieval's own backward
carries to the query and the keys with the reference's key-value semantics;
for idw that gradient also carries the direct terms of the same form
(lam (k - q), lam = dS u sigma, sent as dS sigma), and the rest of the part
with the sub-scores held fixed (idw 2 U gbar for the query and -2 gbar sum_t U
for the keys, from the forward-time key values; dot dS gbar) goes to the
query and the keys directly.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _lib
from ..embedding_bag import _aligned, _require_device
from ..product_keys import SCORE_TYPES, share_distance_products

ME_MAX_N_KEYS = 1024
_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def supported(n_keys: int, dtype: torch.dtype, score_type: str) -> bool:
    """Whether the kernels take these sizes (otherwise the caller keeps the
    torch-op address loss)."""
    return 1 <= n_keys <= ME_MAX_N_KEYS and dtype in _DTYPES and score_type in SCORE_TYPES


def _workspace(tokens, heads, n, dev):
    ws_bytes = int(_lib.load().pkm_me_grad_workspace_size(tokens, heads, n))
    return torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)


class _AddrKeyGrad(torch.autograd.Function):
    """(entropies [2] float32, not differentiable; the key table's gradient of
    w * (-H_1 - H_2)) from the queries, the key table and the sub-score
    matrices with their top-k lists. Batched operands are [2 heads, ...] with
    batch b = 2h + c (head h, half c), the key table's row blocks."""

    @staticmethod
    def forward(ctx, query, keys, s1, s2, sel1, sel2, heads, topk, weight, score_type, share_with=None):
        ctx.set_materialize_grads(False)
        tokens, n = s1.shape[0], s1.shape[-1]
        half = keys.shape[1]
        idw = score_type == "idw"
        dev = s1.device
        s1c, s2c = _aligned(s1), _aligned(s2)
        sel1c, sel2c = sel1.contiguous(), sel2.contiguous()
        # half-queries [2 heads, tokens, half] and keys [2 heads, n, half], float32
        qb = query.detach().float().reshape(tokens, 2 * heads, half).transpose(0, 1)
        kf = keys.detach().float().reshape(2 * heads, n, half)
        qq = kk = dots = None
        if idw:
            # the reference path's mm-based distance operands (|q|^2 + |k|^2 - 2 <q, k>)
            dots = torch.bmm(qb, kf.transpose(1, 2).contiguous())
            qq = (qb * qb).sum(-1).contiguous()
            kk = (kf * kf).sum(-1).contiguous()
            if share_with is not None:
                # the retrieval's backward needs the same products of the same operands
                share_distance_products(share_with, dots, qq, kk)
        entropy = torch.empty(2, device=dev, dtype=torch.float32)
        coef = torch.empty((2 * heads, tokens, n), device=dev, dtype=torch.float32)
        avec = torch.empty((2, n), device=dev, dtype=torch.float32)
        pbar = torch.empty((2, n), device=dev, dtype=torch.float32)
        cs = torch.empty((2 * heads, n), device=dev, dtype=torch.float32) if idw else None  # sum_t U_tj
        ws = _workspace(tokens, heads, n, dev)
        _lib.call("pkm_me_grad_fwd", _lib.ptr(s1c), _lib.ptr(s2c), _lib.ptr(sel1c), _lib.ptr(sel2c),
                  _lib.dtype_code(s1c), tokens, heads, n, topk, _lib.SCORE_CODES[score_type], float(weight),
                  _lib.ptr(qq), _lib.ptr(kk), _lib.ptr(dots), _lib.ptr(entropy), _lib.ptr(coef), _lib.ptr(avec),
                  _lib.ptr(pbar), _lib.ptr(cs), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
        g = torch.bmm(coef.transpose(1, 2), qb)
        if idw:
            g = 2.0 * (g - kf * cs[:, :, None])
        ctx.heads, ctx.topk, ctx.weight, ctx.score_type = heads, topk, float(weight), score_type
        ctx.query_shape, ctx.query_dtype, ctx.keys_dtype = query.shape, query.dtype, keys.dtype
        # idw: the forward-time key values (kf is a copy when the keys are not float32; the
        # caller may store updated weights into a float32 table in place before the backward)
        kf_saved = (kf.clone() if kf.data_ptr() == keys.data_ptr() else kf) if idw else None
        ctx.save_for_backward(qb, kf_saved, s1c, s2c, sel1c, sel2c, avec, pbar, cs, qq, kk, dots)
        ctx.mark_non_differentiable(entropy)
        return entropy, g.reshape(keys.shape).to(keys.dtype)

    @staticmethod
    def backward(ctx, _d_entropy, gbar):
        qb, kf, s1, s2, sel1, sel2, avec, pbar, cs, qq, kk, dots = ctx.saved_tensors
        heads, topk, score_type = ctx.heads, ctx.topk, ctx.score_type
        nones = (None,) * 7
        if gbar is None:
            return (None, None, None, None) + nones
        tokens, n = s1.shape[0], s1.shape[-1]
        half = qb.shape[-1]
        idw = score_type == "idw"
        dev = s1.device
        gb = gbar.float().reshape(2 * heads, n, half)
        qg = torch.bmm(qb, gb.transpose(1, 2).contiguous())  # <q_t, gbar_j>
        kg = (kf * gb).sum(-1).contiguous() if idw else None  # <k_j, gbar_j>
        adot = torch.empty((2, n), device=dev, dtype=torch.float32)
        d_s1 = torch.empty_like(s1)
        d_s2 = torch.empty_like(s2)
        ul = torch.empty((2 * heads, tokens, n), device=dev, dtype=torch.float32)
        ws = _workspace(tokens, heads, n, dev)
        _lib.call("pkm_me_grad_hvp", _lib.ptr(s1), _lib.ptr(s2), _lib.ptr(sel1), _lib.ptr(sel2),
                  _lib.dtype_code(s1), tokens, heads, n, topk, _lib.SCORE_CODES[score_type], ctx.weight,
                  _lib.ptr(qq), _lib.ptr(kk), _lib.ptr(kg), _lib.ptr(dots), _lib.ptr(qg), _lib.ptr(avec),
                  _lib.ptr(pbar), _lib.ptr(adot), _lib.ptr(d_s1), _lib.ptr(d_s2), _lib.ptr(ul), _lib.ptr(ws),
                  ws.numel(), _lib.stream_of(dev))
        # the direct terms left beside the sub-scores' gradient: idw 2 U gbar and -2 gbar colsum(U),
        # dot dS gbar
        d_query = d_keys = None
        if ctx.needs_input_grad[0]:
            dq = torch.bmm(ul, gb)
            if idw:
                dq = 2.0 * dq
            d_query = dq.transpose(0, 1).reshape(ctx.query_shape).to(ctx.query_dtype)
        if idw and ctx.needs_input_grad[1]:
            d_keys = (-2.0 * gb * cs[:, :, None]).reshape(2 * heads * n, half).to(ctx.keys_dtype)
        return (d_query, d_keys, d_s1 if ctx.needs_input_grad[2] else None,
                d_s2 if ctx.needs_input_grad[3] else None) + nones


def addr_loss_and_key_grad(query: torch.Tensor, keys: torch.Tensor, s1: torch.Tensor, s2: torch.Tensor,
                           sel1: torch.Tensor, sel2: torch.Tensor, heads: int, topk: int, weight: float,
                           score_type: str, create_graph: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(addr_loss, d addr_loss / d keys) of the "me" address loss:

      addr_loss = weight * (-1.0 * H(s1) + -1.0 * H(s2)),  in the scores' dtype,
      H(s)      = -sum_j pbar_j log(pbar_j + 1e-8),  pbar = mean over rows of
                  softmax(s masked to each row's topk best, float32)

    as compute_addr_loss (fwpkm/fwpkm.py:233-264) and
    torch.autograd.grad(addr_loss, keys, create_graph=create_graph).

    query: [tokens, heads, k_dim] (the retrieval's queries); keys [2 heads n,
    k_dim / 2] (the table the sub-scores were taken from); s1, s2 [tokens,
    heads, n] the sub-score matrices and sel1, sel2 [tokens, heads, topk] the
    per-half top-k lists of that retrieval (best first). The loss is not
    differentiable (it is only logged); the gradient is, when create_graph.
    """
    _require_device(query, keys, s1, s2, sel1, sel2)
    st = score_type if score_type in SCORE_TYPES else None
    if st is None:
        raise NotImplementedError(f"addr_loss_and_key_grad: score type {score_type}")
    if create_graph:
        entropy, g = _AddrKeyGrad.apply(query, keys, s1, s2, sel1, sel2, heads, topk, weight, st, s1)
    else:
        with torch.no_grad():
            entropy, g = _AddrKeyGrad.apply(query.detach(), keys.detach(), s1.detach(), s2.detach(), sel1, sel2,
                                            heads, topk, weight, st, s1)
    h1, h2 = entropy[0].to(s1.dtype), entropy[1].to(s1.dtype)
    return weight * (-1.0 * h1 + -1.0 * h2), g


__all__ = ["addr_loss_and_key_grad", "supported", "ME_MAX_N_KEYS"]
