"""GPU parity of the fused FwPKM values update (pkm_fw_sgd_update) against
oracle.fw_update, which applies the reference's ATen ops in the same dtype on
the CPU: every step rounds to the dtype in the same order, so the results are
bit-exact. Its autograd (create_graph updates) is checked against torch's
autograd of the reference expression, and FastWeightProductKeyMemory.update_fw
against the oracle end to end."""
from __future__ import annotations

from collections import OrderedDict

import pytest
import torch

from modelos_amd.fwpkm.fwpkm import sgd_value_update
from oracle import fw_update as ref
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu


def _inputs(K, D, B, L, dtype, seed):
    g = gen(seed)
    p = torch.randn((K, D), generator=g).to(dtype)
    grad = (torch.randn((K, D), generator=g) * 1e-4).to(dtype)
    idx = torch.randint(0, max(K - 3, 1), (B, L), generator=g)  # the last rows never indexed
    return p, grad, idx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("clip,wd", [(False, 0.0), (True, 0.0), (True, 0.01), (False, 0.1)],
                         ids=["plain", "clip", "clip-wd", "wd"])
def test_matches_oracle_bit_exact(device, dtype, clip, wd):
    K, D, B, L = 4096, 256, 64, 96
    p, grad, idx = _inputs(K, D, B, L, dtype, seed=3)
    scale, lr = 64 * 256 * 32 * 4, 0.05
    new, gs = sgd_value_update(p.to(device), grad.to(device), idx.to(device), scale, lr, wd, clip)
    e_new, e_gs = ref.sgd_value_update(p, grad, idx, scale, lr, wd, clip)
    torch.cuda.synchronize()
    assert torch.equal(gs.cpu(), e_gs)
    assert torch.equal(new.cpu(), e_new)


def test_large_table_layer_shape(device):
    """2^18 x 1024 bf16 (the fast-weight table size), 16384 x 256 lookups."""
    K, D = 1 << 18, 1024
    gd = torch.Generator(device=device).manual_seed(4)
    p = torch.randn((K, D), generator=gd, device=device).to(torch.bfloat16)
    grad = (torch.randn((K, D), generator=gd, device=device) * 1e-5).to(torch.bfloat16)
    idx = torch.randint(0, K, (16384, 256), generator=gd, device=device)
    new, gs = sgd_value_update(p, grad, idx, 16384 * 1024 * 32 * 8, 0.01, 0.0, True)
    rows = torch.randint(0, K, (256,), generator=gen(5)).to(device)
    # the oracle's steps on the sampled rows, with their counts from the full index set
    cnt = torch.bincount(idx.view(-1), minlength=K)[rows].cpu().to(torch.bfloat16)
    cnt[cnt == 0] = 1.0
    e_gs = (grad[rows].cpu() * (16384 * 1024 * 32 * 8)) / cnt[:, None]
    e_new = p[rows].cpu() - 0.01 * (torch.clamp(e_gs, -1, 1) + 0.0 * p[rows].cpu())
    torch.cuda.synchronize()
    assert torch.equal(gs[rows].cpu(), e_gs)
    assert torch.equal(new[rows].cpu(), e_new)


@pytest.mark.parametrize("clip", [False, True], ids=["plain", "clip"])
def test_autograd_matches_reference_expression(device, clip):
    K, D, B, L = 512, 64, 16, 40
    p, grad, idx = _inputs(K, D, B, L, torch.float32, seed=6)
    grad = grad * 1e4  # values of order one, so clipping engages
    scale, lr, wd = 3.0, 0.1, 0.05
    d_new = torch.randn((K, D), generator=gen(7))
    d_gs = torch.randn((K, D), generator=gen(8))

    def run(fn):
        pp = p.to(device).requires_grad_(True)
        gg = grad.to(device).requires_grad_(True)
        new, gs = fn(pp, gg)
        torch.autograd.backward([new, gs], [d_new.to(device), d_gs.to(device)])
        return pp.grad.cpu(), gg.grad.cpu()

    got = run(lambda a, b: sgd_value_update(a, b, idx.to(device), scale, lr, wd, clip))
    exp = run(lambda a, b: ref.sgd_value_update(a, b, idx.to(device), scale, lr, wd, clip))
    torch.cuda.synchronize()
    assert_rel_close(got[0], exp[0], REL_TOL[torch.float32], "d values")
    assert_rel_close(got[1], exp[1], REL_TOL[torch.float32], "d grad")


def _fw_module(clip):
    """A FastWeightProductKeyMemory whose update_fw (fwpkm.py:274-367) is
    called directly: 2 heads, top-8, value dim 64, 2^12 slots."""
    from modelos_amd.fwpkm.fwpkm import FastWeightProductKeyMemory

    m = FastWeightProductKeyMemory(mem_k_dim=32, mem_v_dim=64, mem_heads=2, mem_topk=8, mem_n_subkeys=64,
                                   learning_rate=0.5, weight_decay=0.01, grad_clip=clip)
    return m.eval()


@pytest.mark.parametrize("clip", [False, True], ids=["plain", "clip"])
def test_update_fw_end_to_end(device, clip):
    g = gen(9)
    V = torch.randn((4096, 64), generator=g).to(device).requires_grad_(True)
    Kp = torch.randn((10, 4), generator=g).to(device).requires_grad_(True)
    idx = torch.randint(0, 250, (12, 16), generator=g).to(device)
    w = torch.randn((12, 16), generator=g).to(device)
    target = torch.randn((12, 64), generator=g).to(device)
    hyp = (V[idx] * w[..., None]).sum(1)
    mem_loss = ((hyp - target) ** 2).mean(-1).mean()
    addr_loss = (Kp ** 2).sum()
    # oracle: the same gradients (taken first: update_fw frees the graph), then the reference's steps
    gv = torch.autograd.grad(0.5 * mem_loss, V, retain_graph=True)[0]
    gk = torch.autograd.grad(addr_loss, Kp, retain_graph=True)[0]
    mod = _fw_module(clip)
    params = OrderedDict([("keys", Kp), ("values", V)])
    upd, grads = mod.update_fw(params, 12, idx, mem_loss, addr_loss)
    e_v, e_gv = ref.sgd_value_update(V.detach().cpu(), gv.cpu(), idx.cpu(), 12 * 64 * 8 * 2, 0.5, 0.01, clip)
    e_gk = torch.clamp(gk, -1, 1) if clip else gk
    e_k = Kp.detach() - 0.5 * (e_gk + 0.01 * Kp.detach())
    torch.cuda.synchronize()
    assert list(upd.keys()) == ["keys", "values"]
    assert torch.equal(upd["values"].detach().cpu(), e_v)
    assert torch.equal(grads[1].detach().cpu(), e_gv)
    assert torch.equal(upd["keys"].detach(), e_k)


def _fused_case(device, dtype, D, clip, wd, seed, K=3000, BT=96, HK=32):
    """A values table, a bag over it and a stand-in memory loss whose gradient
    w.r.t. the bag output drives the step: (values, idx, psw, hyp, loss)."""
    from modelos_amd.fwpkm.xformer_embeddingbag_grad_wrapper import xformers_embedding_bag

    g = gen(seed)
    values = (torch.randn((K, D), generator=g) * 0.1).to(dtype).to(device).requires_grad_(True)
    idx = torch.randint(0, K - 5, (BT, HK), generator=g).to(device)  # the last rows untouched
    idx[0, :4] = 7  # a row looked up several times by one bag
    logits = torch.randn((BT, HK), generator=g).to(device).requires_grad_(True)
    psw = torch.softmax(logits, -1).to(dtype)
    target = torch.randn((BT, D), generator=g).to(dtype).to(device)
    hyp = xformers_embedding_bag(indices=idx, weight=values, per_sample_weights=psw)
    loss = torch.nn.functional.mse_loss(hyp, target, reduction="none").mean(-1).mean()
    return values, idx, logits, psw, hyp, loss


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("D", [256, 1024, 64])
@pytest.mark.parametrize("clip,wd", [(False, 0.0), (True, 0.0), (True, 0.01)], ids=["plain", "clip", "clip-wd"])
def test_fused_values_step_equals_separate_passes(device, dtype, D, clip, wd):
    """The values step fused into the value backward (pkm_eb_bwd_sgd) gives the
    separate passes' results bit for bit (table gradient, then
    pkm_fw_sgd_update), and the same outer gradients of a loss on the new
    values (its double backward, pkm_eb_bwd2_sgd, against autograd through
    EmbeddingBagBW and the step's backward) within the dtype's tolerance."""
    from modelos_amd.fwpkm.fwpkm import _FusedValueStep

    scale, lr = 96 * D * 8 * 4, 0.1
    outs = []
    for fused in (False, True):
        values, idx, logits, psw, hyp, loss = _fused_case(device, dtype, D, clip, wd, seed=9)
        if fused:
            (d_hyp,) = torch.autograd.grad(0.5 * loss, hyp, create_graph=True)
            new, gs, sumsq = _FusedValueStep.apply(values, idx, psw, d_hyp, scale, lr, wd, clip)
        else:
            (gv,) = torch.autograd.grad(0.5 * loss, values, create_graph=True)
            new, gs = sgd_value_update(values, gv, idx, scale, lr, wd, clip)
            sumsq = None
        # an outer loss on the updated table, read through a second bag
        w2 = torch.linspace(-1, 1, D, device=device, dtype=torch.float32)
        outer = (new.float()[idx[:, :8]].sum(1) * w2).sum() + 1e-3 * (gs.float() * w2).sum()
        outer.backward()
        torch.cuda.synchronize()
        outs.append((new.detach(), gs.detach(), sumsq, values.grad, logits.grad))
    (n0, g0, _, dv0, dl0), (n1, g1, ss1, dv1, dl1) = outs
    assert torch.equal(n0, n1) and torch.equal(g0, g1)
    assert_rel_close(ss1.view(-1, 1).sqrt().cpu(), g0.float().pow(2).sum(1, keepdim=True).sqrt().cpu(), 1e-5,
                     "row norms")
    tol = REL_TOL[dtype]
    assert_rel_close(dv1, dv0, tol, "d_values")
    assert_rel_close(dl1, dl0, 1e-4 if dtype == torch.float32 else 5e-2, "d_logits")
