"""Drop-in for the reference's pkm/memory.py: the product-key memory layer.

HashingMemory keeps the reference's constructor arguments, parameter names
and shapes (so state dicts load unchanged), reset_parameters, and its forward
contract x [B, T, C] -> (out [B, T, output_dim], indices [B, T, heads * knn]).
On gfx950 HIP kernels:

  * get_indices: sub-key scores on MFMA and the per-half top-k in one kernel,
    the cartesian top-k in a second one for bf16 scores (in the same kernel
    for float32) (modelos_amd.product_keys); the backward works
    from the nonzeros of the sub-score gradient (dq gathered, dK on MFMA);
  * the value read: the weighted embedding bag (xFormerEmbeddingBag);
  * the glue around them: the query RMSNorm, the score softmax, the swilu
    gate and the Linears' bias gradients, one kernel each way.

The Linear products run on the vendor BLAS (their weight gradients as a
split-K batched product).

Reference: pkm/memory.py:15-28 (ProductKeyArgs), :37-248 (HashingMemory),
:250-289 (get_indices), :292-349 (QueryMLP).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from logging import getLogger
from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from .. import _lib
from ..embedding_bag import _aligned
from ..product_keys import check_supported, product_key_topk, score_softmax
from ..rmsnorm import QueryRMSNorm
from ..swilu import swilu_gate
from .colwise_embedding_bag import xFormerEmbeddingBag


def _weight_grad_splits(rows: int, out_features: int, in_features: int) -> int:
    """Row splits for the weight gradient g^T x of a Linear over `rows`
    inputs: enough that (256 x 256 output tiles) x splits covers the GPU's 256
    CUs, each split at least 2048 rows."""
    tiles = max(1, (out_features // 256) * (in_features // 256))
    s = 1
    while s * 2 * tiles <= 256 and rows % (s * 2) == 0 and rows // (s * 2) >= 2048:
        s *= 2
    return s


class _Linear(torch.autograd.Function):
    """F.linear with the same gradients as nn.Linear's autograd, the weight
    gradient g^T x of a 2-D bf16/fp16 input on the GPU formed as a split-K
    batched product (float32 partials, summed in split order, rounded once):
    the plain product has only (out/256)(in/256) output tiles for K = rows.

    Under torch.autocast the operands are cast to the autocast dtype as
    autocast casts F.linear's, the products run in that dtype, and each
    gradient is returned in its own input's dtype (fp32 master weights get
    fp32 gradients), as nn.Linear's autograd does."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.dtypes = (x.dtype, weight.dtype, bias.dtype if bias is not None else None)
        dev = x.device.type
        if torch.is_autocast_enabled(dev):
            dt = torch.get_autocast_dtype(dev)
            x, weight = x.to(dt), weight.to(dt)
            bias = bias.to(dt) if bias is not None else None
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        with torch.autocast(dev, enabled=False):
            return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        x_dt, w_dt, b_dt = ctx.dtypes
        g = g.to(x.dtype).contiguous()
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            gx = (g @ weight).to(x_dt)
        if ctx.needs_input_grad[1]:
            rows, (out_f, in_f) = x.shape[0], weight.shape
            s = 1
            if g.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and x.is_contiguous():
                s = _weight_grad_splits(rows, out_f, in_f)
            if s > 1:
                part = torch.bmm(g.view(s, rows // s, out_f).transpose(1, 2), x.view(s, rows // s, in_f),
                                 out_dtype=torch.float32)
                gw = _column_sum(part.view(s, out_f * in_f), weight.dtype).view(out_f, in_f)
            else:
                gw = g.t() @ x
            gw = gw.to(w_dt)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            gb = _column_sum(g).to(b_dt)
        return gx, gw, gb


def _column_sum(g: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """g.sum(0) of a 2-D matrix in out_dtype (default g's). On the GPU always
    pkm_column_sum (float32 / bfloat16 / float16, float32 sums over fixed row
    blocks, deterministic); other dtypes raise. CPU tensors (the wrapper's
    host-side tests: the layer itself has no CPU path) use torch's sum."""
    out_dtype = out_dtype or g.dtype
    if not g.is_cuda:
        return g.sum(0).to(out_dtype)
    if g.dim() != 2 or g.dtype not in _lib.DTYPE_CODES or out_dtype not in _lib.DTYPE_CODES:
        raise NotImplementedError(f"column sum of a {g.dim()}-D {g.dtype} matrix into {out_dtype} is not supported")
    rows, cols = g.shape
    out = torch.empty(cols, dtype=out_dtype, device=g.device)
    if cols == 0:
        return out
    g = g.contiguous()
    ws_bytes = int(_lib.load().pkm_column_sum_workspace_size(rows, cols))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=g.device)
    _lib.call("pkm_column_sum", _lib.ptr(g), rows, cols, _lib.dtype_code(g), _lib.DTYPE_CODES[out_dtype],
              _lib.ptr(out), _lib.ptr(ws), ws_bytes, _lib.stream_of(g.device))
    return out


def _linear(layer: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """layer(x) for a 2-D x, through _Linear."""
    return _Linear.apply(x, layer.weight, layer.bias)

logger = getLogger()


@dataclass
class ProductKeyArgs:
    """Model-config block of the PKM layers (pkm/memory.py:15-28)."""

    is_enabled: bool = False
    layers: str = ""
    mem_n_keys: int = 1024
    mem_heads: int = 4
    mem_knn: int = 32
    mem_share_values: bool = True
    mem_k_dim: int = 512
    mem_v_dim: int = -1
    swilu_projection: bool = True
    value_fixed_lr: Optional[float] = 0.001
    mem_gated: bool = False
    peer_variant: bool = False


class AttrDict(dict):
    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.__dict__ = self


class HashingMemory(nn.Module):
    """Product-key memory read (pkm/memory.py:37-248)."""

    VALUES = None
    EVAL_MEMORY = True

    def __init__(
        self,
        input_dim,
        output_dim,
        value_fixed_lr=0.001,
        mem_k_dim=512,
        mem_v_dim=-1,
        mem_heads=4,
        mem_knn=32,
        mem_share_values=True,
        mem_n_keys=1024,
        mem_query_bias=True,
        mem_query_batchnorm=False,
        mem_query_rmsnorm=True,
        mem_gated=False,
        mem_input_dropout=0.0,
        mem_query_dropout=0.0,
        mem_value_dropout=0.0,
        peer_variant=False,
        swilu_projection=True,
    ):
        # argument checks of the reference (memory.py:71-95)
        assert mem_k_dim >= 2 and mem_k_dim % 2 == 0
        assert 0 <= mem_input_dropout < 1 and 0 <= mem_query_dropout < 1 and 0 <= mem_value_dropout < 1
        assert not (peer_variant and mem_v_dim > 0), (
            "Cannot use PEER variant with a value dimension different from the input dimension (mem_v_dim=-1)"
        )
        assert mem_heads >= 2
        if mem_query_batchnorm:
            logger.warning(
                "WARNING: if you use batch normalization, be sure that you use batches of sentences with the same "
                "size at training time. Otherwise, the padding token will result in incorrect mean/variance "
                "estimations in the BatchNorm layer."
            )
        assert not (mem_query_batchnorm and mem_query_rmsnorm), "Cannot use both batchnorm and rmsnorm"
        value_width = None if peer_variant else (mem_v_dim if mem_v_dim > 0 else output_dim)
        check_supported(mem_n_keys, mem_k_dim, mem_knn, value_width, "HashingMemory")
        super().__init__()
        self.use_peer_variant = peer_variant
        self.input_dim = input_dim
        self.output_dim = output_dim
        self.size = mem_n_keys**2
        self.k_dim = mem_k_dim
        self.v_dim = mem_v_dim if mem_v_dim > 0 else output_dim
        self.swilu_proj = swilu_projection
        self.v_proj = mem_v_dim > 0 or self.swilu_proj
        self.heads = mem_heads
        self.knn = mem_knn
        self.input_dropout = mem_input_dropout
        self.query_dropout = mem_query_dropout
        self.value_dropout = mem_value_dropout

        # keys: [2 * heads * n_keys, k_dim / 2]; key (h, c, i) is row (2h + c) * n_keys + i
        self.keys = nn.Parameter(torch.zeros(2 * self.heads * int(self.size**0.5), self.k_dim // 2))

        self.mem_share_values = mem_share_values
        self.original = not self.mem_share_values or HashingMemory.VALUES is None
        if self.original:
            if not self.use_peer_variant:
                self.values = xFormerEmbeddingBag(self.size, self.v_dim)
            else:
                self.values_u = nn.Embedding(self.size, self.v_dim)
                self.values_v = nn.Embedding(self.size, self.v_dim)
        else:
            if not self.use_peer_variant:
                self.values = None
            else:
                self.values_u = None
                self.values_v = None
        self.value_fixed_lr = value_fixed_lr

        if self.v_proj:
            proj_input = mem_v_dim
            if self.swilu_proj and proj_input < 0:
                proj_input = output_dim
            self.value_proj = nn.Linear(proj_input, output_dim)
        if self.swilu_proj:
            self.swilu_projection = nn.Linear(self.input_dim, proj_input)
        self.gating = nn.Linear(input_dim, 1) if mem_gated else None

        self.query_proj = QueryMLP(
            self.input_dim,
            self.heads,
            self.k_dim,
            (self.input_dim, self.heads * self.k_dim),
            bias=mem_query_bias,
            batchnorm=mem_query_batchnorm,
            rmsnorm=mem_query_rmsnorm,
        )

    def reset_parameters(self, init_std=None, factor=1.0):
        """Initialisation of the reference (memory.py:169-188)."""
        bound = 1 / math.sqrt(self.k_dim)
        nn.init.uniform_(self.keys, a=-bound, b=bound)
        if self.original:
            if not self.use_peer_variant:
                nn.init.normal_(self.values.weight, mean=0, std=self.v_dim**-0.5)
            else:
                nn.init.normal_(self.values_u.weight, mean=0, std=self.v_dim**-0.5)
                nn.init.normal_(self.values_v.weight, mean=0, std=self.v_dim**-0.5)
        nn.init.xavier_uniform_(self.query_proj.query_mlps[0].weight)
        if self.v_proj:
            nn.init.normal_(self.value_proj.weight, mean=0, std=self.output_dim**-0.5)
        if self.swilu_proj:
            nn.init.normal_(self.swilu_projection.weight, mean=0, std=self.output_dim**-0.5)
        if self.gating is not None:
            nn.init.normal_(self.gating.weight, mean=0, std=self.input_dim**-0.5)

    def forward(self, input):
        """x [B, T, C] -> (out [B, T, output_dim], indices [B, T, heads * knn]) (memory.py:190-248)."""
        B, T, C = input.shape
        input = input.view(-1, self.input_dim)
        bs = input.shape[0]
        input = F.dropout(input, p=self.input_dropout, training=self.training)
        query = self.query_proj(input)  # [bs * heads, k_dim]
        query = F.dropout(query, p=self.query_dropout, training=self.training)
        assert query.shape == (bs * self.heads, self.k_dim)

        knn = self.knn
        scores, indices = self.get_indices(query, knn)  # [bs * heads, knn] each

        if not self.training and HashingMemory.EVAL_MEMORY:
            # usage statistics, eval mode only (memory.py:212-215)
            self.last_indices = indices.view(bs, self.heads, knn).detach().cpu()
            self.last_scores = scores.view(bs, self.heads, knn).detach().cpu().float()

        # softmax over each head's knn scores in float32 (memory.py:218)
        scores = score_softmax(scores)
        indices = indices.view(bs, self.heads * knn)
        scores = scores.view(bs, self.heads * knn)

        if not self.use_peer_variant:
            output = self.values(indices, scores)  # [bs, v_dim]
            if self.v_proj and not self.swilu_proj:
                output = _linear(self.value_proj, output)
            if self.swilu_proj:
                output = _linear(self.value_proj, swilu_gate(output, _linear(self.swilu_projection, input)))
        else:
            # PEER variant (memory.py:231-237): per-slot expert vectors
            u = self.values_u(indices)  # [bs, heads * knn, v_dim]
            x = torch.bmm(u, input.unsqueeze(-1)).squeeze(-1)
            x = F.gelu(x) * scores
            v = self.values_v(indices)
            output = torch.bmm(x.unsqueeze(1), v).squeeze(1)

        output = F.dropout(output, p=self.value_dropout, training=self.training)  # [bs, output width]
        if self.gating:
            output = F.sigmoid(_linear(self.gating, input)) * output
        return output.view(B, T, -1), indices.view(B, T, -1)

    def get_indices(self, query, knn):
        """(scores, indices) [bs * heads, knn]: the best knn product keys per
        (token, head), best first (memory.py:250-289), from the fused scoring
        and selection kernels of pkm_score_topk; equal scores are ordered by
        the smaller sub-key position."""
        assert query.dim() == 2 and query.size(1) == self.k_dim
        return product_key_topk(query, self.keys, self.heads, knn, "dot")


class QueryMLP(nn.Module):
    """Query network: Linear (+ReLU chain) then BatchNorm / RMSNorm (memory.py:292-349)."""

    def __init__(self, input_dim, heads, k_dim, sizes, bias=False, batchnorm=False, rmsnorm=False):
        super().__init__()
        self.input_dim = input_dim
        self.heads = heads
        self.k_dim = k_dim
        self.sizes = sizes
        assert sizes[0] == input_dim
        assert sizes[-1] == (heads * k_dim)
        self.query_mlps = QueryMLP.mlp(list(sizes), bias=bias)
        if batchnorm:
            self.norm = nn.BatchNorm1d(sizes[-1], affine=True, eps=1e-6, momentum=0.1)
        elif rmsnorm:
            # Qwen3RMSNorm (memory.py:311) on the fused HIP kernels
            self.norm = QueryRMSNorm(sizes[-1], eps=1e-6)
        else:
            self.norm = None

    @staticmethod
    def mlp(sizes, bias=True):
        assert len(sizes) >= 2
        layers = []
        n = len(sizes) - 1
        for i in range(n):
            layers.append(nn.Linear(sizes[i], sizes[i + 1], bias=bias))
            if i < n - 1:
                layers.append(nn.ReLU())
        return nn.Sequential(*layers)

    def forward(self, input):
        assert input.shape[-1] == self.input_dim
        input = input.contiguous().view(-1, self.input_dim) if input.dim() > 2 else input
        bs = len(input)
        query = input
        for layer in self.query_mlps:
            query = _linear(layer, query) if isinstance(layer, nn.Linear) else layer(query)
        if self.norm is not None:
            query = self.norm(query)
        assert query.shape == (bs, self.heads * self.k_dim)
        return query.view(bs * self.heads, self.k_dim)
