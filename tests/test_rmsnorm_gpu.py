"""Fused query RMS norm (pkm_rmsnorm_fwd / pkm_rmsnorm_bwd) against a plain
PyTorch reference of the same op sequence (Qwen3RMSNorm, pkm/memory.py:311),
on the GPU in float32 and bfloat16, and against the float64 CPU oracle."""
from __future__ import annotations

import pytest
import torch

from modelos_amd.rmsnorm import QueryRMSNorm, rms_norm
from oracle import rmsnorm as ref
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu

SHAPES = [
    (37, 4096),  # query rows of the layer (8 heads x k_dim 512)
    (5, 2048),
    (3, 8192),  # 16 heads x 512: rows too long to hold in registers
    (64, 512),
    (129, 1024),  # more than two 64-row weight-gradient blocks, ragged
]


def _inputs(N, D, dtype, seed):
    g = gen(seed)
    x = torch.randn((N, D), generator=g).to(dtype)
    w = (1.0 + 0.1 * torch.randn((D,), generator=g)).to(dtype)
    dy = torch.randn((N, D), generator=g).to(dtype)
    return x, w, dy


def _run(fn, x, w, dy):
    xg = x.clone().requires_grad_()
    wg = w.clone().requires_grad_()
    y = fn(xg, wg)
    y.backward(dy)
    return y.detach(), xg.grad, wg.grad


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_matches_torch_reference(device, shape, dtype):
    N, D = shape
    x, w, dy = (t.to(device) for t in _inputs(N, D, dtype, 1))
    got = _run(lambda a, b: rms_norm(a, b, 1e-6), x, w, dy)
    exp = _run(lambda a, b: ref.rms_norm(a, b, 1e-6), x, w, dy)
    torch.cuda.synchronize()
    for a, e, what in zip(got, exp, ("y", "dx", "dweight")):
        assert a.dtype == dtype
        assert_rel_close(a, e, REL_TOL[dtype], what)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_matches_float64_oracle(device, dtype):
    x, w, dy = _inputs(48, 4096, dtype, 2)
    got = _run(lambda a, b: rms_norm(a, b, 1e-6), x.to(device), w.to(device), dy.to(device))
    exp = _run(lambda a, b: ref.rms_norm(a, b, 1e-6), x.double(), w.double(), dy.double())
    for a, e, what in zip(got, exp, ("y", "dx", "dweight")):
        assert_rel_close(a, e, REL_TOL[dtype], what)


def test_layer_shape_and_determinism(device):
    x, w, dy = (t.to(device) for t in _inputs(16384, 4096, torch.bfloat16, 3))
    a = _run(lambda p, q: rms_norm(p, q, 1e-6), x, w, dy)
    b = _run(lambda p, q: rms_norm(p, q, 1e-6), x, w, dy)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    e = _run(lambda p, q: ref.rms_norm(p, q, 1e-6), x[:512], w, dy[:512])
    assert_rel_close(a[0][:512], e[0], REL_TOL[torch.bfloat16], "y rows")
    assert_rel_close(a[1][:512], e[1], REL_TOL[torch.bfloat16], "dx rows")
    full_dw = _run(lambda p, q: ref.rms_norm(p, q, 1e-6), x, w, dy)[2]
    assert_rel_close(a[2], full_dw, REL_TOL[torch.bfloat16], "dweight")


def test_empty_rows(device):
    x = torch.empty((0, 4096), dtype=torch.bfloat16, device=device, requires_grad=True)
    w = torch.ones(4096, dtype=torch.bfloat16, device=device, requires_grad=True)
    y = rms_norm(x, w, 1e-6)
    y.sum().backward()
    assert y.shape == (0, 4096)
    assert torch.equal(w.grad, torch.zeros_like(w))


def test_module_is_a_qwen3_rmsnorm_drop_in(device):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    a, b = QueryRMSNorm(4096, eps=1e-6), Qwen3RMSNorm(4096, eps=1e-6)
    assert list(a.state_dict()) == list(b.state_dict()) and a.variance_epsilon == b.variance_epsilon
    b.load_state_dict(a.state_dict())
    x = torch.randn((7, 4096), generator=gen(4)).to(device)
    torch.testing.assert_close(a.to(device)(x), b.to(device)(x), rtol=1e-5, atol=1e-6)


def test_cpu_tensors_raise():
    with pytest.raises(RuntimeError, match="no CPU path"):
        rms_norm(torch.ones(2, 8), torch.ones(8), 1e-6)


def test_unsupported_inputs_raise(device):
    """No silent torch path: other dtype combinations and row widths raise."""
    x = torch.randn((4, 4096), device=device).to(torch.bfloat16)
    with pytest.raises(NotImplementedError):
        rms_norm(x, torch.ones(4096, device=device), 1e-6)  # float32 weight, bfloat16 rows
    with pytest.raises(NotImplementedError):
        rms_norm(torch.randn((4, 4094), device=device), torch.ones(4094, device=device), 1e-6)
    with pytest.raises(NotImplementedError):
        rms_norm(x.half(), torch.ones(4096, device=device).half(), 1e-6)
