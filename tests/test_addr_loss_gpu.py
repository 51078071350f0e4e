"""Marginal-entropy address loss kernels (pkm_me_grad_fwd / pkm_me_grad_hvp)
through modelos_amd.fwpkm.marginal_entropy (GPU).

  * against float64 autograd on the CPU of the reference's expressions
    (oracle/fwpkm.py: sub_scores, marginal_entropy; fwpkm/fwpkm.py:117-147,
    233-264, 853-869): the loss, the key table's gradient, and the gradient
    of <gbar, that gradient> with respect to the query and the keys (the
    double backward), float32 inputs, the kernel's own sub-scores deciding
    the masks; shapes with n_keys and half not multiples of 64 and key tables
    with duplicated rows (exact ties at the top-k threshold: the mask keeps
    more than topk entries);
  * against the module's torch-op address loss (compute_addr_loss and
    autograd, create_graph), float32 and bfloat16, the same retrieval;
  * bitwise reproducible;
  * the fast-weight module with and without the kernels: the same outputs,
    losses and outer gradients.
"""
from __future__ import annotations

import pytest
import torch

from oracle import fwpkm as ofw
from tests.helpers import assert_norm_close, assert_rel_close, gen

pytestmark = pytest.mark.gpu

# (tokens, heads, n_keys, k_dim, topk, duplicated key rows)
SHAPES = [
    (40, 4, 128, 64, 8, False),
    (37, 2, 100, 140, 5, False),
    (48, 2, 64, 32, 8, True),
    (512, 4, 512, 256, 16, False),
]


def _ids(v):
    return str(v).replace("torch.", "")


def _inputs(tokens, heads, n, k_dim, dup, dtype, seed=0):
    g = gen(seed)
    half = k_dim // 2
    keys = (torch.rand((2 * heads * n, half), generator=g) * 2 - 1) * k_dim**-0.5
    if dup:
        # every key of each (head, half) block has a twin: equal scores, ties at any threshold
        kb = keys.view(2 * heads, n, half)
        kb[:, 1::2] = kb[:, 0::2]
    q = torch.randn((tokens, heads, k_dim), generator=g) * 0.3
    gbar = torch.randn((2 * heads * n, half), generator=g)
    return q.to(dtype), keys.to(dtype), gbar


def _retrieve(q, keys, heads, topk, score_type):
    from modelos_amd.product_keys import product_key_topk

    st = "idw" if score_type == "idw" else "dot"
    _, _, i1, i2, s1, s2 = product_key_topk(q, keys, heads, topk, st, sub_outputs=True)
    return s1, s2, i1, i2


def _kernel_path(q, keys, heads, topk, weight, score_type, gbar):
    from modelos_amd.fwpkm.marginal_entropy import addr_loss_and_key_grad

    q = q.detach().requires_grad_(True)
    keys = keys.detach().requires_grad_(True)
    s1, s2, i1, i2 = _retrieve(q, keys, heads, topk, score_type)
    loss, g = addr_loss_and_key_grad(q, keys, s1, s2, i1, i2, heads, topk, weight,
                                     "idw" if score_type == "idw" else "dot", create_graph=True)
    dq, dk = torch.autograd.grad((g.float() * gbar).sum(), (q, keys))
    return loss.detach(), g.detach(), dq, dk, (s1.detach(), s2.detach())


def _torch_path(q, keys, heads, topk, weight, score_type, gbar, n, k_dim):
    """The module's torch-op address loss (compute_addr_loss) and autograd."""
    from modelos_amd.fwpkm.fwpkm import FastWeightProductKeyMemory

    mem = FastWeightProductKeyMemory(mem_k_dim=k_dim, mem_v_dim=16, mem_heads=heads, mem_topk=topk,
                                     mem_n_subkeys=n, qk_score_type=score_type, addr_loss="me",
                                     addr_loss_weight=weight)
    q = q.detach().requires_grad_(True)
    keys = keys.detach().requires_grad_(True)
    s1, s2, i1, i2 = _retrieve(q, keys, heads, topk, score_type)
    loss = mem.compute_addr_loss(i1, i2, s1, s2)
    (g,) = torch.autograd.grad(loss, keys, create_graph=True)
    dq, dk = torch.autograd.grad((g.float() * gbar).sum(), (q, keys))
    return loss.detach(), g.detach(), dq, dk


def _fp64(q, keys, heads, topk, weight, score_type, gbar, n, k_dim, sel_scores):
    cfg = ofw.FwConfig(heads=heads, k_dim=k_dim, v_dim=16, topk=topk, subsize=n, score_type=score_type,
                       addr_loss_weight=weight)
    q64 = q.detach().cpu().double().requires_grad_(True)
    k64 = keys.detach().cpu().double().requires_grad_(True)
    s1, s2 = ofw.sub_scores(q64, k64, cfg)
    loss = ofw.addr_loss({"s1": s1, "s2": s2}, cfg, sel_scores=[s.cpu() for s in sel_scores])
    (g,) = torch.autograd.grad(loss, k64, create_graph=True)
    dq, dk = torch.autograd.grad((g * gbar.double()).sum(), (q64, k64))
    return loss.detach(), g.detach(), dq, dk


@pytest.mark.parametrize("score_type", ["idw", "dot_product"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s[:5])) + ("-dup" if s[5] else ""))
def test_float32_against_float64(shape, score_type, device):
    tokens, heads, n, k_dim, topk, dup = shape
    q, keys, gbar = _inputs(tokens, heads, n, k_dim, dup, torch.float32)
    weight = 0.7
    loss, g, dq, dk, sub = _kernel_path(q.to(device), keys.to(device), heads, topk, weight, score_type,
                                        gbar.to(device))
    e_loss, e_g, e_dq, e_dk = _fp64(q, keys, heads, topk, weight, score_type, gbar, n, k_dim, sub)
    assert_rel_close(loss, e_loss, 1e-5, "addr_loss")
    # sums over tokens with cancellation: 2-norm relative error
    assert_norm_close(g, e_g, 1e-5, "key gradient")
    assert_norm_close(dq, e_dq, 1e-4, "d query")
    assert_norm_close(dk, e_dk, 1e-4, "d keys")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=_ids)
@pytest.mark.parametrize("score_type", ["idw", "dot_product"])
def test_matches_torch_op_path(dtype, score_type, device):
    tokens, heads, n, k_dim, topk = 256, 4, 256, 128, 8
    q, keys, gbar = _inputs(tokens, heads, n, k_dim, False, dtype, seed=3)
    q, keys, gbar = q.to(device), keys.to(device), gbar.to(device)
    a = _kernel_path(q, keys, heads, topk, 1.0, score_type, gbar)
    b = _torch_path(q, keys, heads, topk, 1.0, score_type, gbar, n, k_dim)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert_rel_close(a[0], b[0], tol, "addr_loss")
    for x, y, what in zip(a[1:4], b[1:4], ("key gradient", "d query", "d keys")):
        assert_norm_close(x, y, tol if what == "key gradient" else 10 * tol, what)


def test_reproducible(device):
    q, keys, gbar = _inputs(512, 4, 512, 256, False, torch.float32, seed=9)
    q, keys, gbar = q.to(device), keys.to(device), gbar.to(device)
    r1 = _kernel_path(q, keys, 4, 16, 1.0, "idw", gbar)
    r2 = _kernel_path(q, keys, 4, 16, 1.0, "idw", gbar)
    for x, y in zip(r1[:4], r2[:4]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("score_type", ["idw", "dot_product"])
def test_module_with_and_without_kernels(score_type, device, monkeypatch):
    from modelos_amd.fwpkm.fwpkm import FastWeightProductKeyMemory

    kw = dict(mem_k_dim=64, mem_v_dim=64, mem_heads=2, mem_topk=8, mem_n_subkeys=64, lookahead=0,
              qk_score_type=score_type, learning_rate=0.3, addr_loss_weight=0.5)
    g = gen(11)
    x = torch.randn((2, 96, 2 * 64), generator=g) * 0.3
    ref_v = torch.randn((2, 96, 64), generator=g)
    dout = torch.randn((2, 96, 64), generator=g)
    torch.manual_seed(0)
    base = FastWeightProductKeyMemory(**kw)
    base.reset_parameters()

    def run(kernels: bool):
        mem = FastWeightProductKeyMemory(**kw).to(device).train()
        with torch.no_grad():
            mem.keys.copy_(base.keys)
            mem.values.copy_(base.values)
        if not kernels:
            monkeypatch.setattr(mem, "_addr_kernels", lambda *a, **k: False)
        xd = x.to(device).requires_grad_(True)
        out = mem(q=xd, ref_v=ref_v.to(device), gates=None, chunk_size=32)
        out["output"].backward(dout.to(device))
        return out, xd.grad, mem.keys.grad, mem.values.grad, mem.keys.detach().clone()

    a, b = run(True), run(False)
    assert torch.equal(a[0]["indices"], b[0]["indices"])
    assert_rel_close(a[0]["output"], b[0]["output"], 1e-5, "output")
    assert_rel_close(a[0]["addr_loss"], b[0]["addr_loss"], 1e-5, "addr_loss")
    assert_rel_close(a[4], b[4], 1e-5, "final keys")
    for x_, y_, what in zip(a[1:4], b[1:4], ("dx", "dkeys", "dvalues")):
        assert_norm_close(x_, y_, 1e-4, what)
