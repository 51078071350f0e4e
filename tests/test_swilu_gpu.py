"""GPU parity of the fused SwiLU gate (pkm_swilu_fwd / pkm_swilu_bwd) against
the reference expression `e * F.silu(s)` (pkm/memory.py:229) and its autograd,
run by torch on the same device: same float32 math and rounding points, so the
outputs and both gradients are expected bit for bit."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from modelos_amd.swilu import swilu_gate
from tests.helpers import gen

pytestmark = pytest.mark.gpu


def _run(fn, e, s, dh):
    ee = e.clone().requires_grad_(True)
    ss = s.clone().requires_grad_(True)
    h = fn(ee, ss)
    h.backward(dh)
    return h.detach(), ee.grad, ss.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("shape", [(16384, 1024), (37, 13), (5,), (3, 8)], ids=["layer", "ragged", "tiny", "one-vector"])
def test_matches_torch(device, dtype, shape):
    g = gen(7)
    e = (torch.randn(shape, generator=g) * 0.5).to(dtype).to(device)
    s = (torch.randn(shape, generator=g) * 3).to(dtype).to(device)
    dh = torch.randn(shape, generator=g).to(dtype).to(device)
    got = _run(swilu_gate, e, s, dh)
    exp = _run(lambda a, b: a * F.silu(b), e, s, dh)
    torch.cuda.synchronize()
    for name, x, y in zip(("h", "de", "ds"), got, exp):
        assert x.dtype == y.dtype and x.shape == y.shape
        assert torch.equal(x, y), f"{name}: max abs diff {(x.float() - y.float()).abs().max().item():.3e}"


def test_extreme_inputs(device):
    """Large |s| (exp overflow / underflow), zeros, signed zeros, infinities."""
    s = torch.tensor([-1e4, -90.0, -20.0, -0.0, 0.0, 1e-30, 20.0, 90.0, 1e4, float("inf"), float("-inf"), 3.0,
                      -3.0, 0.5, -0.5, 7.0], device=device)
    e = torch.linspace(-2, 2, s.numel(), device=device)
    dh = torch.linspace(1, -1, s.numel(), device=device)
    got = _run(swilu_gate, e, s, dh)
    exp = _run(lambda a, b: a * F.silu(b), e, s, dh)
    torch.cuda.synchronize()
    for name, x, y in zip(("h", "de", "ds"), got, exp):
        assert torch.equal(x.nan_to_num(7.0), y.nan_to_num(7.0)), name


def test_empty(device):
    e = torch.zeros((0, 8), device=device, dtype=torch.bfloat16)
    h = swilu_gate(e, e)
    assert h.shape == (0, 8)
