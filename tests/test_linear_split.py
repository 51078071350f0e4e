"""The layer's Linear wrapper: same forward and gradients as nn.Linear's
autograd; on the GPU the bf16 weight gradient is a split-K product with
float32 partials (checked against float64 at the bf16 tolerance)."""
from __future__ import annotations

import pytest
import torch
from torch import nn

from modelos_amd.pkm.memory import _linear, _weight_grad_splits
from tests.helpers import REL_TOL, assert_rel_close, gen


def _grads(layer, x, g, fn):
    layer.zero_grad(set_to_none=True)
    xx = x.clone().requires_grad_(True)
    y = fn(layer, xx)
    y.backward(g)
    return y.detach(), xx.grad, layer.weight.grad, layer.bias.grad


def test_matches_nn_linear_cpu_fp32():
    torch.manual_seed(0)
    layer = nn.Linear(64, 48)
    x = torch.randn((300, 64), generator=gen(1))
    g = torch.randn((300, 48), generator=gen(2))
    a = _grads(layer, x, g, lambda m, v: m(v))
    b = _grads(layer, x, g, _linear)
    for u, v in zip(a, b):
        assert torch.allclose(u, v, rtol=1e-6, atol=1e-6)


def test_split_heuristic():
    assert _weight_grad_splits(16384, 1024, 1024) == 8
    assert _weight_grad_splits(16384, 4096, 1024) == 4
    assert _weight_grad_splits(4096, 1024, 1024) == 2
    assert _weight_grad_splits(3000, 1024, 1024) == 1  # below 2 x 2048 rows
    assert _weight_grad_splits(16384 + 2, 1024, 1024) == 2  # rows must divide evenly


@pytest.mark.gpu
@pytest.mark.parametrize("rows,in_f,out_f", [(16384, 1024, 1024), (16384, 1024, 4096), (8192, 256, 512)])
def test_split_k_weight_grad_gpu(device, rows, in_f, out_f):
    torch.manual_seed(0)
    layer = nn.Linear(in_f, out_f).to(device).to(torch.bfloat16)
    x = torch.randn((rows, in_f), device=device).to(torch.bfloat16)
    g = torch.randn((rows, out_f), device=device).to(torch.bfloat16)
    y, gx, gw, gb = _grads(layer, x, g, _linear)
    y0, gx0, gw0, gb0 = _grads(layer, x, g, lambda m, v: m(v))
    torch.cuda.synchronize()
    assert torch.equal(y, y0) and torch.equal(gx, gx0)  # same products as nn.Linear
    e_gw = g.double().t() @ x.double()
    assert_rel_close(gw, e_gw, REL_TOL[torch.bfloat16], "grad_weight")
    assert_rel_close(gb, g.double().sum(0), REL_TOL[torch.bfloat16], "grad_bias")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(16384, 4096), (16384, 1024), (1000, 24), (33, 8), (1, 64), (500, 1001),
                                       (40, 3), (2, 7)])
def test_column_sum_gpu(device, dtype, rows, cols):
    """pkm_column_sum against a float64 sum, deterministic run to run."""
    from modelos_amd.pkm.memory import _column_sum

    g = torch.randn((rows, cols), generator=gen(3)).to(dtype).to(device)
    a = _column_sum(g)
    b = _column_sum(g)
    torch.cuda.synchronize()
    assert a.dtype == dtype and a.shape == (cols,)
    assert torch.equal(a, b)
    assert_rel_close(a, g.double().sum(0), REL_TOL[dtype], "column sum")


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [8, 32, 33, 200])
def test_column_sum_float32_to_bf16(device, rows):
    """float32 input summed into a bfloat16 output (the split-K partials of a
    weight gradient): one rounding of the float32 sum."""
    from modelos_amd.pkm.memory import _column_sum

    g = torch.randn((rows, 4096), generator=gen(4)).to(device)
    a = _column_sum(g, torch.bfloat16)
    torch.cuda.synchronize()
    assert a.dtype == torch.bfloat16
    assert_rel_close(a, g.double().sum(0), REL_TOL[torch.bfloat16], "column sum")


@pytest.mark.gpu
def test_column_sum_no_rows(device):
    from modelos_amd.pkm.memory import _column_sum

    g = torch.zeros((0, 64), device=device, dtype=torch.bfloat16)
    assert not bool(_column_sum(g).any())


def test_matches_nn_linear_under_autocast_cpu():
    """fp32 master weights under autocast(bf16): the product runs in bf16 and
    every gradient comes back in its input's dtype, exactly as nn.Linear's."""
    torch.manual_seed(0)
    layer = nn.Linear(64, 48)
    x = torch.randn((40, 64), generator=gen(3))
    g = torch.randn((40, 48), generator=gen(4))

    def run(fn):
        layer.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        with torch.autocast("cpu", dtype=torch.bfloat16):
            y = fn(layer, xx)
        y.float().backward(g)
        return y.detach(), xx.grad, layer.weight.grad, layer.bias.grad

    a = run(lambda m, v: m(v))
    b = run(_linear)
    assert b[0].dtype == torch.bfloat16
    assert [t.dtype for t in b[1:]] == [torch.float32] * 3
    for u, v in zip(a, b):
        assert u.dtype == v.dtype and torch.equal(u, v)
