"""Drop-in for the reference's pkm/xformer_embeddingbag.py, on gfx950 HIP kernels.

Same public names, argument meaning, return conventions and assertions as the
reference module; the Triton kernels are replaced by libpkm_hip.so:

- embedding_bag_triton (reference :116-138)       -> pkm_eb_fwd
- embedding_bag_bw_rev_indices (reference :331-386) -> pkm_eb_bwd (deterministic)
- embedding_bag_bw2 (reference :209-258)           -> pkm_eb_bwd as well (the
  reference's atomics/lock variants compute the same gradients; its "lock"
  variant returns an all-zero weight gradient, a bug not reproduced here)
- xFormersEmbeddingBag / xformers_embedding_bag (reference :389-438)

DTensor inputs are unwrapped with to_local() and the results re-wrapped like
the reference does (weight grad Shard(-1), psw grad Partial(sum)); no
collective is issued here.

Difference by design: the reference falls back to F.embedding_bag for CPU
tensors (:436-437). This module has no CPU path and raises for CPU tensors.
"""
from __future__ import annotations

from typing import Tuple

import torch
from torch.distributed.tensor import DTensor, Partial, Shard

from .. import embedding_bag as _eb


def embedding_bag_triton(indices: torch.Tensor, weight: torch.Tensor, per_sample_weights: torch.Tensor) -> torch.Tensor:
    """Forward gather; name kept from the reference (:116)."""
    distributed = isinstance(indices, DTensor)
    if distributed:
        mesh = weight.device_mesh
        indices = indices.to_local()
        weight = weight.to_local()
        per_sample_weights = per_sample_weights.to_local()
    out = _eb.eb_forward(indices, weight, per_sample_weights)
    if distributed:
        out = DTensor.from_local(out, mesh, (Shard(-1),), run_check=False)
    return out


def embedding_bag_bw_rev_indices(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: torch.Tensor,
    gradient: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns (weight.grad, per_sample_weights.grad); reference :331-386."""
    distributed = isinstance(indices, DTensor)
    if distributed:
        mesh = weight.device_mesh
        indices = indices.to_local()
        weight = weight.to_local()
        per_sample_weights = per_sample_weights.to_local()
        gradient = gradient.to_local()
    K, _ = weight.shape
    B, bag_size = indices.shape
    assert B * bag_size < 2**31, "bags * bag_size must be < 2**31"
    weight_grad, per_sample_weights_grad = _eb.eb_backward(indices, weight, per_sample_weights, gradient)
    if distributed:
        weight_grad = DTensor.from_local(weight_grad, mesh, (Shard(-1),), run_check=False)
        per_sample_weights_grad = DTensor.from_local(
            per_sample_weights_grad, mesh, (Partial(reduce_op="sum"),), run_check=False
        )
    return weight_grad, per_sample_weights_grad


def embedding_bag_bw2(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: torch.Tensor,
    gradient: torch.Tensor,
    use_atomics: bool,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Reference :209-258 (atomics / lock bag-centric backward). Same gradients,
    computed by the deterministic kernel."""
    assert indices.is_contiguous()
    assert weight.is_contiguous()
    assert per_sample_weights.is_contiguous()
    assert gradient.is_contiguous()
    return embedding_bag_bw_rev_indices(indices, weight, per_sample_weights, gradient)


class xFormersEmbeddingBag(torch.autograd.Function):
    """Reference :389-425: forward gather, backward (None, gW, gpsw, None)."""

    @staticmethod
    def forward(ctx, indices, weight, per_sample_weights, bw_algo):
        ctx.save_for_backward(indices, weight, per_sample_weights)
        ctx.bw_algo = bw_algo
        return embedding_bag_triton(indices, weight, per_sample_weights)

    @staticmethod
    def backward(ctx, gradient):
        indices, weight, per_sample_weights = ctx.saved_tensors
        if ctx.bw_algo in ["lock", "atomics"]:
            weight_g, per_sample_weights_g = embedding_bag_bw2(
                indices, weight, per_sample_weights, gradient.contiguous(), use_atomics=ctx.bw_algo == "atomics"
            )
        else:
            assert ctx.bw_algo == "reverse_indices"
            weight_g, per_sample_weights_g = embedding_bag_bw_rev_indices(indices, weight, per_sample_weights, gradient)
        return None, weight_g, per_sample_weights_g, None


def xformers_embedding_bag(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: torch.Tensor,
    mode: str = "sum",
    bw_algo: str = "reverse_indices",
) -> torch.Tensor:
    """Reference :428-438 (mode must be "sum")."""
    assert mode == "sum"
    return xFormersEmbeddingBag.apply(indices, weight, per_sample_weights, bw_algo)


class CustomEmbeddingBagFunction(torch.autograd.Function):
    """Reference :35-84, the pure-PyTorch comparator; here it runs the same HIP
    kernels (backward_chunks only changed the reference's memory use)."""

    @staticmethod
    def forward(ctx, indices, weight, per_sample_weights, mode="sum", backward_chunks=1):
        assert mode == "sum", "CustomEmbeddingBagFunction only implements SUM mode for now."
        assert indices.size(0) % backward_chunks == 0
        ctx.save_for_backward(indices, weight, per_sample_weights)
        return _eb.eb_forward(indices, weight, per_sample_weights)

    @staticmethod
    def backward(ctx, grad_output):
        indices, weight, per_sample_weights = ctx.saved_tensors
        gw, gpsw = _eb.eb_backward(indices, weight, per_sample_weights, grad_output)
        return None, gw, gpsw, None, None


def custom_embedding_bag_function(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: torch.Tensor,
    mode: str = "sum",
) -> torch.Tensor:
    assert mode == "sum"
    return CustomEmbeddingBagFunction.apply(indices, weight, per_sample_weights)
