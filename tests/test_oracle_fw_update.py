"""Pins oracle.fw_update (the FwPKM values update, fwpkm/fwpkm.py:334-365,
266-272) against closed forms and a brute-force count."""
from __future__ import annotations

import torch

from oracle import fw_update as ref
from tests.helpers import gen


def test_counts_brute_force():
    g = gen(1)
    idx = torch.randint(0, 50, (7, 33), generator=g)
    c = ref.row_counts(idx, 60)
    brute = torch.tensor([int((idx == r).sum()) for r in range(60)])
    assert torch.equal(c, brute)


def test_closed_form_without_clip_or_decay():
    g = gen(2)
    K, D = 40, 16
    p = torch.randn((K, D), generator=g, dtype=torch.float64)
    grad = torch.randn((K, D), generator=g, dtype=torch.float64)
    idx = torch.randint(0, 30, (5, 12), generator=g)  # rows 30..39 never indexed
    scale, lr = 5 * 16 * 4 * 3, 0.01
    new, gs = ref.sgd_value_update(p, grad, idx, scale, lr, 0.0, False)
    cnt = torch.tensor([max(int((idx == r).sum()), 1) for r in range(K)], dtype=torch.float64)
    e_gs = grad * scale / cnt[:, None]
    assert torch.allclose(gs, e_gs, rtol=1e-14, atol=0)
    assert torch.allclose(new, p - lr * e_gs, rtol=1e-14, atol=1e-15)
    assert torch.equal(gs[30:], grad[30:] * scale)  # untouched rows divide by one


def test_clip_and_decay():
    p = torch.tensor([[1.0, -2.0, 0.5, 4.0]], dtype=torch.float64)
    grad = torch.tensor([[3.0, -3.0, 0.25, 0.0]], dtype=torch.float64)
    idx = torch.tensor([[0, 0]])  # count 2
    new, gs = ref.sgd_value_update(p, grad, idx, 2.0, 0.1, 0.5, True)
    assert torch.equal(gs, grad)  # 2 * g / 2
    e_new = p - 0.1 * (torch.tensor([[1.0, -1.0, 0.25, 0.0]], dtype=torch.float64) + 0.5 * p)
    assert torch.allclose(new, e_new, rtol=1e-15, atol=1e-16)
