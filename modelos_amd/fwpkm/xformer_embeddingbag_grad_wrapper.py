"""Drop-in for the reference's fwpkm/xformer_embeddingbag_grad_wrapper.py.

Autograd structure kept from the reference (grad_wrapper:13-163) so fwpkm's
in-context update can differentiate through the first-order backward:

- _XEmbeddingBagFn.forward(weight, indices, psw, bw_kernel): the bag gather,
  here the HIP forward kernel (the reference materialises index_select + sum,
  :98-103);
- _XEmbeddingBagFn.backward: calls bw_kernel (indices, weight, psw, grad) ->
  (grad_weight, grad_psw) and wraps grad_weight in EmbeddingBagBW so the
  graph has a node carrying its VJP (:127-155);
- EmbeddingBagBW.backward(g_bar): the double backward, here one fused HIP
  kernel (the reference materialises a [B, bag, D] gather, :55-74).

psw may be None (unweighted bag) everywhere, as in the reference.
"""
from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch
from torch.autograd import Function

from .. import embedding_bag as _eb
from .xformer_embeddingbag_legacy import embedding_bag_bw_rev_indices


class EmbeddingBagBW(Function):
    @staticmethod
    def forward(
        ctx,
        indices: torch.Tensor,  # [B, bag], long
        per_sample_weights: Optional[torch.Tensor],  # [B, bag] or None
        grad_output: torch.Tensor,  # [B, D]
        num_embeddings: int,  # K
        embedding_dim: int,  # D
        fast_grad_weight: torch.Tensor,  # [K, D], from the first-order kernel
    ) -> torch.Tensor:
        if per_sample_weights is None:
            ctx.has_psw = False
            ctx.save_for_backward(
                indices, torch.empty(0, device=grad_output.device, dtype=grad_output.dtype), grad_output
            )
        else:
            ctx.has_psw = True
            ctx.save_for_backward(indices, per_sample_weights, grad_output)
        ctx.num_embeddings = num_embeddings
        ctx.embedding_dim = embedding_dim
        return fast_grad_weight

    @staticmethod
    def backward(ctx, g_bar: torch.Tensor):
        """Grads for (indices, per_sample_weights, grad_output, K, D, fast_grad_weight):
        d_a[b,j] = <g_bar[idx[b,j]], grad_output[b]>, d_grad_output[b] = sum_j a[b,j] g_bar[idx[b,j]]."""
        idx, a_saved, g = ctx.saved_tensors
        a = a_saved if ctx.has_psw else None
        d_grad_output, d_a = _eb.eb_double_backward(idx, a, g, g_bar)
        return (None, d_a, d_grad_output, None, None, None)


class _XEmbeddingBagFn(Function):
    @staticmethod
    def forward(
        ctx,
        weight: torch.Tensor,  # [K, D]
        indices: torch.Tensor,  # [B, bag], long
        per_sample_weights: Optional[torch.Tensor],  # [B, bag] or None
        bw_kernel: Callable[
            [torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor], Tuple[torch.Tensor, torch.Tensor]
        ],
    ) -> torch.Tensor:
        assert indices.dtype == torch.long
        K, D = weight.shape
        out = _eb.eb_forward(indices, weight, per_sample_weights)
        ctx.save_for_backward(
            weight,
            indices,
            per_sample_weights
            if per_sample_weights is not None
            else torch.empty(0, device=weight.device, dtype=weight.dtype),
        )
        ctx.has_psw = per_sample_weights is not None
        ctx.K, ctx.D = K, D
        ctx.bw_kernel = bw_kernel
        # a table handle whose other consumer parks its gradient for this backward to add into
        ctx.sink = getattr(weight, "_pkm_grad_sink", None)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        weight, indices, a_saved = ctx.saved_tensors
        K, D = ctx.K, ctx.D
        a = a_saved if ctx.has_psw else None
        res = None
        if ctx.sink is not None and ctx.bw_kernel is _bw_kernel and not torch.is_grad_enabled():
            pending = ctx.sink.take()
            if pending is not None:
                res = _eb.eb_backward_into(indices, weight, a, grad_output, pending)
                if res is None:
                    ctx.sink.pending = pending  # no accumulating kernel here: the fan-out node adds it
        # first-order kernel: not differentiable; EmbeddingBagBW carries the VJP
        with torch.no_grad():
            weight_grad_fast, psw_grad_fast = res if res is not None else ctx.bw_kernel(indices, weight, a,
                                                                                          grad_output)
        grad_weight = EmbeddingBagBW.apply(indices, a if ctx.has_psw else None, grad_output, K, D, weight_grad_fast)
        grad_psw = psw_grad_fast if ctx.has_psw else None
        return grad_weight, None, grad_psw, None


def _bw_kernel(indices, weight, per_sample_weights, gradient):
    """bw_kernel with psw=None support (unweighted bag)."""
    if per_sample_weights is None:
        return _eb.eb_backward(indices, weight, None, gradient)
    return embedding_bag_bw_rev_indices(indices, weight, per_sample_weights, gradient)


def xformers_embedding_bag(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: torch.Tensor,
) -> torch.Tensor:
    """Reference grad_wrapper:158-163 (weight first in apply, no mode argument)."""
    return _XEmbeddingBagFn.apply(weight, indices, per_sample_weights, _bw_kernel)
