"""Drop-in for the reference's pkm/colwise_embedding_bag.py (value-table module).

xFormerEmbeddingBag keeps the reference's parameter name (`weight`, [size, dim],
zero-initialised: colwise_embedding_bag.py:28-31), its repr, its
torch.compiler.disable wrapper and its DTensor gradient-averaging trick
(:36-49). The lookup runs on the HIP kernels.

ColwiseEmbeddingBag (the tensor-parallel ParallelStyle, :52-114) is not part of
this single-GPU build.
"""
from __future__ import annotations

import torch
import torch.nn as nn
from torch.distributed.tensor import DTensor

from .xformer_embeddingbag import xformers_embedding_bag


class xFormerEmbeddingBag(nn.Module):
    def __init__(self, size, dim):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(size, dim))

    def __repr__(self):
        return f"xFormerEmbeddingBag(num_embeddings={self.weight.size(0)}, embedding_dim={self.weight.size(1)})"

    @torch.compiler.disable(recursive=True)
    def forward(self, indices, scores):
        if isinstance(self.weight, DTensor):
            weight = self.weight.to_local()
            num_shards = self.weight.device_mesh.size()
            if num_shards > 1:
                # gradients are averaged over shards rather than summed (reference :41-44)
                grad_scale = 1 / num_shards
                weight = weight * grad_scale + (weight * (1 - grad_scale)).detach()
        else:
            weight = self.weight
        return xformers_embedding_bag(indices, weight, per_sample_weights=scores, mode="sum")
