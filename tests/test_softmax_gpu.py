"""GPU parity of the score softmax (pkm_softmax_fwd / pkm_softmax_bwd)
against the reference expression F.softmax(scores.float(), -1).type_as(scores)
(pkm/memory.py:218) and its autograd, run by torch on the same device. The
kernels sum in column order (torch's softmax in a reduction tree), so the
float32 results agree to rounding: 1e-5 (f32) / 2e-2 (bf16) relative."""
from __future__ import annotations

import pytest
import torch

from modelos_amd import _lib
from modelos_amd.product_keys import score_softmax
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu


def _run(fn, x, dy):
    xx = x.clone().requires_grad_(True)
    y = fn(xx)
    y.backward(dy)
    return y.detach(), xx.grad


def _ref(x):
    return torch.softmax(x.float(), dim=-1).type_as(x)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("shape", [(131072, 32), (300, 64), (77, 7), (5, 1), (3, 4, 33), (101, 8), (99, 16), (50, 4)],
                         ids=["layer", "k64", "k7", "k1", "3d-k33", "k8", "k16", "k4"])
def test_matches_torch(device, dtype, shape):
    g = gen(11)
    x = (torch.randn(shape, generator=g) * 4).to(dtype).to(device)
    dy = torch.randn(shape, generator=g).to(dtype).to(device)
    y, dx = _run(score_softmax, x, dy)
    e_y, e_dx = _run(_ref, x, dy)
    torch.cuda.synchronize()
    assert y.dtype == dtype and dx.dtype == dtype
    assert_rel_close(y, e_y, REL_TOL[dtype], "y")
    assert_rel_close(dx, e_dx, REL_TOL[dtype], "dx")
    # rows sum to one (float32 probabilities before the rounding)
    assert_rel_close(y.double().sum(-1), torch.ones(shape[:-1], dtype=torch.float64), 5e-2 if dtype == torch.bfloat16 else 1e-5, "row sums")


def test_equal_and_extreme_scores(device):
    x = torch.tensor([[0.0] * 32, [1e4] + [-1e4] * 31, [float("-inf")] + [0.0] * 31], device=device)
    dy = torch.randn(x.shape, generator=gen(12)).to(device)
    y, dx = _run(score_softmax, x, dy)
    e_y, e_dx = _run(_ref, x, dy)
    torch.cuda.synchronize()
    assert_rel_close(y, e_y, 1e-6, "y")
    assert_rel_close(dx, e_dx, 1e-5, "dx")


def test_deterministic_and_limits(device):
    x = torch.randn((1000, 32), generator=gen(13)).to(torch.bfloat16).to(device)
    assert torch.equal(score_softmax(x), score_softmax(x))
    with pytest.raises(_lib.PkmError):
        y = torch.empty((2, 65), device=device)
        _lib.call("pkm_softmax_fwd", _lib.ptr(y), 2, 65, _lib.dtype_code(y), _lib.ptr(y), _lib.stream_of(y.device))
