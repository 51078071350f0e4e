"""Drop-in for the reference's fwpkm/xformer_embeddingbag_legacy.py.

The reference module is a copy of the pkm embedding-bag kernels (legacy:33-227)
plus a pure-PyTorch CPU fallback (_embedding_bag_bw_native, legacy:147-167).
Here every name maps to the same gfx950 kernels as modelos_amd.pkm; there is
no CPU fallback (CPU tensors raise).
"""
from __future__ import annotations

import torch

from ..pkm.xformer_embeddingbag import (  # noqa: F401  (re-exported names of the reference module)
    embedding_bag_bw_rev_indices,
    embedding_bag_triton,
)


class xFormersEmbeddingBag(torch.autograd.Function):
    """Reference legacy:232-255 (no bw_algo argument)."""

    @staticmethod
    def forward(ctx, indices, weight, per_sample_weights):
        ctx.save_for_backward(indices, weight, per_sample_weights)
        return embedding_bag_triton(indices, weight, per_sample_weights)

    @staticmethod
    def backward(ctx, gradient):
        indices, weight, per_sample_weights = ctx.saved_tensors
        weight_g, per_sample_weights_g = embedding_bag_bw_rev_indices(indices, weight, per_sample_weights, gradient)
        return None, weight_g, per_sample_weights_g


def xformers_embedding_bag(indices, weight, per_sample_weights, mode: str = "sum"):
    """Reference legacy:258-263."""
    assert mode == "sum"
    return xFormersEmbeddingBag.apply(indices, weight, per_sample_weights)
