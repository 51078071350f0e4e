"""Query RMS normalisation: CPU restatement (test infrastructure only).

Qwen3RMSNorm as the reference's query network applies it (pkm/memory.py:311,
forward at :341-349; the module's forward casts to float32, takes
pow(2).mean(-1), rsqrt(. + eps), multiplies, casts back and multiplies by the
weight). Autograd through this function gives the reference's gradients.
Pinned against transformers' Qwen3RMSNorm (the library module the reference
instantiates) in tests/test_oracle_rmsnorm.py.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    h = x.to(torch.float32) if x.dtype != torch.float64 else x
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)
