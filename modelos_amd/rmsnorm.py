"""Fused RMS normalisation of the product-key query on the HIP kernels.

`QueryRMSNorm` is the Qwen3RMSNorm the reference's query network applies
(pkm/memory.py:311, 341-349; transformers' Qwen3RMSNorm): same parameter
(`weight`, initialised to ones), same `variance_epsilon`, same forward

    y = weight * (x.float() * rsqrt(mean(x.float()^2, -1) + eps)).to(x.dtype)

and the gradients autograd forms through those ops, in two kernels
(pkm_rmsnorm_fwd / pkm_rmsnorm_bwd) instead of about a dozen float32
elementwise and reduction passes over the [tokens, heads * k_dim] query.
The weight gradient is a deterministic column reduction.

Supported: float32 or bfloat16 input with a weight of the same dtype, rows
of whole 16-byte vectors, on the GPU; anything else raises
NotImplementedError. There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .embedding_bag import _require_device

_FUSED_DTYPES = (torch.float32, torch.bfloat16)


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        D = x.shape[-1]
        x2 = x.contiguous().view(-1, D)
        N = x2.shape[0]
        y = torch.empty_like(x2)
        rstd = torch.empty(N, dtype=torch.float32, device=x.device)
        w = weight.contiguous()
        _lib.call("pkm_rmsnorm_fwd", _lib.ptr(x2), _lib.ptr(w), N, D, _lib.dtype_code(x2), float(eps),
                  _lib.ptr(y), _lib.ptr(rstd), _lib.stream_of(x.device))
        ctx.save_for_backward(x2, w, rstd)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2, w, rstd = ctx.saved_tensors
        N, D = x2.shape
        dy2 = dy.contiguous().view(N, D)
        dx = torch.empty_like(x2)
        dw = torch.empty_like(w)
        lib = _lib.load()
        ws_bytes = lib.pkm_rmsnorm_bwd_workspace_size(N, D)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x2.device)
        _lib.call("pkm_rmsnorm_bwd", _lib.ptr(dy2), _lib.ptr(x2), _lib.ptr(w), _lib.ptr(rstd), N, D,
                  _lib.dtype_code(x2), _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(ws), ws_bytes,
                  _lib.stream_of(x2.device))
        return dx.view(ctx.shape), dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * (x.float() * rsqrt(mean(x.float()^2, -1) + eps)).to(x.dtype) over the last dim."""
    _require_device(x, weight)
    if x.dtype != weight.dtype or x.dtype not in _FUSED_DTYPES or x.shape[-1] % (16 // x.element_size()) != 0:
        raise NotImplementedError(
            f"rms_norm: input {x.dtype} with weight {weight.dtype} over rows of {x.shape[-1]} is not supported "
            "(float32 or bfloat16 input and weight of the same dtype, rows of whole 16-byte vectors are)"
        )
    return _RMSNormFn.apply(x, weight, eps)


class QueryRMSNorm(nn.Module):
    """Drop-in for transformers' Qwen3RMSNorm (parameter `weight`, `variance_epsilon`)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return rms_norm(hidden_states, self.weight, self.variance_epsilon)

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"
