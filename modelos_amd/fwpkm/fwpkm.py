"""Drop-in product-key retrieval for the reference's fast-weight PKM
(fwpkm/fwpkm.py:853-934).

FastWeightProductKeyMemory reads the attributes heads, k_dim, topk, subsize
and qk_score_type ("dot_product" or "idw") in compute_qk_scores/get_indices.
ProductKeyIndexMixin provides both methods with the reference's signatures
and return values on the fused HIP kernel (scores, per-half top-k, cartesian
top-k in one launch), differentiable w.r.t. query and keys, including the
full sub-score matrices the address loss uses (fwpkm.py:117-147, 250-253).
A class using it replaces the two methods, e.g.

    class FastWeightProductKeyMemory(ProductKeyIndexMixin, reference.FastWeightProductKeyMemory): ...

FusedValueUpdateMixin.update_fw is the reference's update_fw (fwpkm.py:274-367)
with the values' step (gradient scaling by the sample count, division by the
bincount of the indices, optional clipping, SGD with weight decay) in one
kernel pass over the [size, v_dim] table instead of about a dozen elementwise
passes; it stays differentiable for the outer loss (create_graph).

The rest of the module (value retrieval through
modelos_amd.fwpkm.xformer_embeddingbag_grad_wrapper) is ordinary torch code
around these drop-ins.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Optional

import torch

from .. import _lib
from ..embedding_bag import _aligned, _require_device
from ..product_keys import product_key_topk

SCORE_TYPES = {"dot_product": "dot", "idw": "idw"}


def _score_type(name: str) -> str:
    try:
        return SCORE_TYPES[name]
    except KeyError:
        raise NotImplementedError(f"QK score type {name} not implemented.") from None


def get_indices(query: torch.Tensor, keys: torch.Tensor, heads: int, k_dim: int, topk: int,
                qk_score_type: str = "dot_product"):
    """fwpkm.py:871-934 as a function. query: [BT, heads, k_dim] (any view with
    that many elements); keys: [heads * 2 * subsize, k_dim // 2].
    Returns scores, indices, topk_indices1, topk_indices2 [BT, heads, topk] and
    scores1, scores2 [BT, heads, subsize]; equal scores are ordered by the
    smaller sub-key position."""
    BT = query.numel() // (heads * k_dim)
    q = query.reshape(BT, heads, k_dim)
    scores, idx, i1, i2, s1, s2 = product_key_topk(q, keys, heads, topk, _score_type(qk_score_type),
                                                   sub_outputs=True)
    return (scores.view(BT, heads, topk), idx.view(BT, heads, topk), i1, i2, s1, s2)


def compute_qk_scores(q: torch.Tensor, k: torch.Tensor, qk_score_type: str = "dot_product") -> torch.Tensor:
    """fwpkm.py:853-869: q [batch, heads, d], k [heads, n_keys, d] -> scores
    [batch, heads, n_keys] (dot product, or -log(1e-3 + squared distance)).
    Dense scores without selection are a plain batched GEMM; this form exists
    for callers of the method itself — get_indices never materialises it
    apart from the sub-score outputs."""
    st = _score_type(qk_score_type)
    _require_device(q, k)
    qh = q.permute(1, 0, 2).contiguous()  # [heads, batch, d]
    dots = torch.bmm(qh, k.transpose(1, 2).contiguous())  # [heads, batch, n_keys]
    if st == "dot":
        return dots.permute(1, 0, 2)
    d2 = (qh * qh).sum(-1, keepdim=True) + (k * k).sum(-1)[:, None, :] - 2.0 * dots
    return (-torch.log(1e-3 + d2.clamp_min(0.0))).permute(1, 0, 2)


class ProductKeyIndexMixin:
    """compute_qk_scores / get_indices of FastWeightProductKeyMemory on the
    HIP kernels (needs self.heads, self.k_dim, self.topk, self.qk_score_type)."""

    def compute_qk_scores(self, q, k):
        return compute_qk_scores(q, k, self.qk_score_type)

    def get_indices(self, query, keys):
        return get_indices(query, keys, self.heads, self.k_dim, self.topk, self.qk_score_type)


class _SgdValueUpdate(torch.autograd.Function):
    """(new values, scaled gradient) of the values' SGD step (pkm_fw_sgd_update)."""

    @staticmethod
    def forward(ctx, p, g, counts, scale, lr, wd, clip):
        p2 = _aligned(p)
        g2 = _aligned(g.to(p.dtype))
        counts = counts.contiguous()
        new = torch.empty_like(p2)
        gs = torch.empty_like(p2)
        K, D = p2.shape
        _lib.call("pkm_fw_sgd_update", _lib.ptr(p2), _lib.ptr(g2), _lib.ptr(counts), K, D, _lib.dtype_code(p2),
                  float(scale), float(lr), float(wd), int(bool(clip)), _lib.ptr(gs), _lib.ptr(new),
                  _lib.stream_of(p2.device))
        ctx.save_for_backward(gs, counts)
        ctx.scale, ctx.lr, ctx.wd, ctx.clip = scale, lr, wd, clip
        return new, gs

    @staticmethod
    def backward(ctx, d_new, d_gs):
        # the reference's autograd through p - lr * (clamp(g * scale / c) + wd * p), op by op
        # (pkm_fw_sgd_update_bwd); only the scaled gradient's own gradient: its two ops
        gs, counts = ctx.saved_tensors
        if d_new is None:
            if d_gs is None or not ctx.needs_input_grad[1]:
                return None, None, None, None, None, None, None
            c = counts.to(gs.dtype)
            c[c == 0] = 1.0
            return None, (d_gs / c.unsqueeze(-1)) * ctx.scale, None, None, None, None, None
        dn = _aligned(d_new.to(gs.dtype))
        dgi = _aligned(d_gs.to(gs.dtype)) if d_gs is not None else None
        d_p = torch.empty_like(gs)
        d_g = torch.empty_like(gs)
        K, D = gs.shape
        _lib.call("pkm_fw_sgd_update_bwd", _lib.ptr(dn), _lib.ptr(dgi), _lib.ptr(gs), _lib.ptr(counts), K, D,
                  _lib.dtype_code(gs), float(ctx.scale), float(ctx.lr), float(ctx.wd), int(bool(ctx.clip)),
                  _lib.ptr(d_p), _lib.ptr(d_g), _lib.stream_of(gs.device))
        return (d_p if ctx.needs_input_grad[0] else None), (d_g if ctx.needs_input_grad[1] else None), \
            None, None, None, None, None


def sgd_value_update(p: torch.Tensor, g: torch.Tensor, indices: torch.Tensor, scale: float, lr: float,
                     weight_decay: float, grad_clip: bool):
    """The values branch of update_fw with the "sgd" optimizer
    (fwpkm.py:334-365, 266-272): returns (p - lr * (clip(g') + wd * p), g')
    with g' = g * scale / max(bincount(indices), 1) per row, both in p's
    dtype. float32 / bfloat16 tables on the GPU."""
    _require_device(p, g, indices)
    if p.dim() != 2 or p.shape != g.shape:
        raise ValueError(f"values and gradient must be the same [size, v_dim], got {tuple(p.shape)}, {tuple(g.shape)}")
    if p.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"values dtype {p.dtype} not supported (float32, bfloat16 are)")
    counts = torch.bincount(indices.reshape(-1), minlength=p.shape[0])
    return _SgdValueUpdate.apply(p, g, counts, scale, lr, weight_decay, grad_clip)


class FusedValueUpdateMixin:
    """update_fw of FastWeightProductKeyMemory (fwpkm.py:274-367) with the
    values' step on pkm_fw_sgd_update; the gradients are formed as the
    reference forms them, and every other parameter takes the reference's
    update_fw_param."""

    def update_fw(self, fw_named_params: OrderedDict, num_samples: int, indices: torch.Tensor,
                  mem_loss: torch.Tensor, addr_loss: Optional[torch.Tensor] = None):
        mem_loss = mem_loss * 0.5
        names = list(fw_named_params.keys())
        if self.mem_grad_to_values_only:
            if addr_loss is not None:
                addr_grads = torch.autograd.grad(addr_loss, fw_named_params.values(), create_graph=self.training,
                                                 allow_unused=True)
            else:
                addr_grads = [None] * len(fw_named_params)
            mem_grads = torch.autograd.grad(mem_loss, fw_named_params["values"], create_graph=self.training)
            grads = [mem_grads[0] if n == "values" else addr_grads[i] for i, n in enumerate(names)]
        else:
            loss = mem_loss if addr_loss is None else mem_loss + addr_loss
            grads = list(torch.autograd.grad(loss, tuple(fw_named_params.values()), create_graph=self.training))
        fused = self.optimizer_type == "sgd"
        scale = num_samples * self.v_dim * self.topk * self.heads
        scaled, updated = [], []
        for n, p, g in zip(names, fw_named_params.values(), grads):
            if n == "values" and fused and g is not None:
                new_p, g_scaled = sgd_value_update(p, g, indices, scale, self.learning_rate, self.weight_decay,
                                                   self.grad_clip)
                scaled.append(g_scaled)
                updated.append(new_p)
                continue
            if n == "values":
                g = g * scale
                binc = torch.bincount(indices.view(-1), minlength=self.size).to(g.dtype)
                binc[binc == 0] = 1.0
                g = g / binc.unsqueeze(-1)
            scaled.append(g)
            gc = torch.clamp(g, min=-1.0, max=1.0) if self.grad_clip else g
            updated.append(self.update_fw_param(p, gc, self.learning_rate, self.weight_decay))
        return OrderedDict(zip(names, updated)), scaled
