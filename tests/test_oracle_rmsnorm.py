"""Pins of the query RMS-norm oracle (oracle/rmsnorm.py) on the CPU: against
transformers' Qwen3RMSNorm, the module the reference instantiates
(pkm/memory.py:311), forward and gradients, and a closed form."""
from __future__ import annotations

import pytest
import torch

from oracle import rmsnorm as ref
from tests.helpers import gen


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_matches_qwen3_rmsnorm(dtype):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    g = gen(0)
    x = torch.randn((9, 64), generator=g, dtype=dtype)
    w = torch.randn((64,), generator=g, dtype=dtype)
    m = Qwen3RMSNorm(64, eps=1e-6).to(dtype)
    with torch.no_grad():
        m.weight.copy_(w)
    x1 = x.clone().requires_grad_()
    y1 = m(x1)
    dy = torch.randn(y1.shape, generator=g, dtype=dtype)
    y1.backward(dy)
    x2 = x.clone().requires_grad_()
    w2 = w.clone().requires_grad_()
    y2 = ref.rms_norm(x2, w2, 1e-6)
    y2.backward(dy)
    # the library casts to float32 even for float64 input; the oracle keeps
    # float64 there (its role as the high-precision reference)
    tol = 1e-6
    torch.testing.assert_close(y2, y1, rtol=tol, atol=tol)
    torch.testing.assert_close(x2.grad, x1.grad, rtol=tol, atol=tol)
    torch.testing.assert_close(w2.grad, m.weight.grad, rtol=tol, atol=tol)


def test_closed_form_constant_rows():
    # a row of equal values c normalises to sign(c) * weight (up to eps)
    x = torch.full((3, 16), -2.0, dtype=torch.float64)
    w = torch.arange(16, dtype=torch.float64)
    y = ref.rms_norm(x, w, 0.0)
    torch.testing.assert_close(y, -w.expand(3, 16), rtol=0, atol=1e-15)
