"""SwiLU gating of the PKM layer's value output on the HIP kernels.

`swilu_gate(e, s)` is `e * F.silu(s)` as HashingMemory.forward applies it
(pkm/memory.py:229): silu in float32 rounded to the tensor dtype, the product
rounded again; its backward forms the gradients autograd takes through the
product and F.silu. One kernel each way (pkm_swilu_fwd / pkm_swilu_bwd)
instead of two forward and three backward elementwise passes.

Supported: e and s of one shape and dtype (float32, bfloat16) on the GPU;
other combinations (float16 among them) use the reference expression (plain
torch ops).
There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from .embedding_bag import _aligned, _require_device

_FUSED_DTYPES = (torch.float32, torch.bfloat16)


class _SwiluFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, e: torch.Tensor, s: torch.Tensor):
        e2 = _aligned(e.contiguous())
        s2 = _aligned(s.contiguous())
        h = torch.empty_like(e2)
        _lib.call("pkm_swilu_fwd", _lib.ptr(e2), _lib.ptr(s2), e2.numel(), _lib.dtype_code(e2), _lib.ptr(h),
                  _lib.stream_of(e2.device))
        ctx.save_for_backward(e2, s2)
        return h

    @staticmethod
    def backward(ctx, dh: torch.Tensor):
        e2, s2 = ctx.saved_tensors
        dh2 = _aligned(dh.contiguous())
        de = torch.empty_like(e2)
        ds = torch.empty_like(s2)
        _lib.call("pkm_swilu_bwd", _lib.ptr(dh2), _lib.ptr(e2), _lib.ptr(s2), e2.numel(), _lib.dtype_code(e2),
                  _lib.ptr(de), _lib.ptr(ds), _lib.stream_of(e2.device))
        return de, ds


def swilu_gate(e: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """e * F.silu(s) (same shape and dtype) with the fused forward and backward."""
    _require_device(e, s)
    if e.shape == s.shape and e.dtype == s.dtype and e.dtype in _FUSED_DTYPES:
        return _SwiluFn.apply(e, s)
    return e * F.silu(s)


__all__ = ["swilu_gate"]
