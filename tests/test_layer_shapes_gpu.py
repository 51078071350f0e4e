"""HashingMemory at the benchmark configurations' own shapes (GPU).

  * the CPU parity configuration: input 1024 -> output 1024, 4 heads, 256 keys
    per half (65,536 slots), k_dim 512, knn 32, value dim 1024, float32,
    BatchNorm query in train mode, keys U(-1/16, 1/16), values
    N(0, 1024^-1/2), x [4, 512, 1024] ~ N(0, 1): output and every gradient
    against the float64 oracle evaluated at the kernel's selection, 1e-5
    (normwise and elementwise);
  * the layer benchmark: 8 x 2048 tokens, 8 heads, 1024 keys per half
    (2^20 slots), k_dim 512, knn 32, value dim 1024, RMSNorm query, swilu,
    bfloat16, reset_parameters init: sampled tokens' output and input
    gradient against the float64 oracle at the kernel's selection (the query
    RMSNorm is per token, so a token's output and input gradient depend on
    that token only); sampled rows of the value table's gradient against
    float64 sums over their lookups of the captured bag-output gradient; the
    key and query-weight gradients against float32 torch products of the
    dense sub-score gradient built from the captured score gradient; and
    the retrieval of sampled tokens bit-exact against the oracle's selection
    from the kernel's sub-scores.
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd.pkm.memory import HashingMemory
from modelos_amd.product_keys import score_topk
from oracle import pkm as ref
from oracle import pkm_layer
from tests.helpers import assert_rel_close, gen

pytestmark = pytest.mark.gpu


def test_cpu_parity_config_layer_fp32(device):
    torch.manual_seed(0)
    kw = dict(input_dim=1024, output_dim=1024, mem_k_dim=512, mem_heads=4, mem_knn=32, mem_n_keys=256,
              mem_query_batchnorm=True, mem_query_rmsnorm=False)
    mem = HashingMemory(**kw)
    mem.reset_parameters()
    g = gen(3)
    with torch.no_grad():
        mem.keys.copy_((torch.rand(mem.keys.shape, generator=g) * 2 - 1) / 16)
        mem.values.weight.copy_(torch.randn(mem.values.weight.shape, generator=g) * 1024**-0.5)
    mem = mem.to(device).train()
    x = torch.randn((4, 512, 1024), generator=g)
    dout = torch.randn((4, 512, 1024), generator=g)
    xd = x.to(device).requires_grad_(True)
    out, idx = mem(xd)
    out.backward(dout.to(device))
    P = {n: p.detach().cpu().double().requires_grad_(True) for n, p in mem.named_parameters()}
    x64 = x.double().requires_grad_(True)
    e_out, _ = pkm_layer.hashing_memory_forward(x64, P, 4, 32, batchnorm=True, idx=idx.cpu().view(-1, 32))
    e_out.backward(dout.double())
    assert_rel_close(out, e_out, 1e-5, "out")
    # the train-mode BatchNorm's backward subtracts batch means: dx entries are differences of sums
    # over the batch, so the elementwise bound applies from a quarter of the maximum
    assert_rel_close(xd.grad, x64.grad, 1e-5, "dx", elem_frac=0.25)
    for name, p in mem.named_parameters():
        atol = 0.0
        if name == "query_proj.query_mlps.0.bias":  # removed by the train-mode BatchNorm: zero up to rounding
            atol = 1e-5 * P["query_proj.query_mlps.0.weight"].grad.abs().max().item()
        # parameter gradients are sums over the 2048 tokens: elementwise from a quarter of the maximum
        assert_rel_close(p.grad, P[name].grad, 1e-5, f"grad {name}", atol, elem_frac=0.25)


def _layer_module(device):
    torch.manual_seed(0)
    mem = HashingMemory(input_dim=1024, output_dim=1024, mem_k_dim=512, mem_heads=8, mem_knn=32, mem_n_keys=1024,
                        mem_query_rmsnorm=True)
    mem.reset_parameters()
    return mem.to(device=device, dtype=torch.bfloat16).train()


def test_layer_benchmark_shape_bf16(device):
    H, knn, n = 8, 32, 1024
    mem = _layer_module(device)
    g = gen(11)
    x = torch.randn((8, 2048, 1024), generator=g).to(torch.bfloat16)
    dout = torch.randn((8, 2048, 1024), generator=g).to(torch.bfloat16)
    captured = {}

    # capture the gradient reaching the selected scores and the bag output
    orig_get, orig_values = mem.get_indices, mem.values.forward

    def get_indices(query, k):
        sc, ix = orig_get(query, k)
        sc.register_hook(lambda gr: captured.__setitem__("d_scores", gr.detach()))
        query.register_hook(lambda gr: captured.__setitem__("d_query", gr.detach()))
        captured["query"] = query.detach()
        return sc, ix

    mem.query_proj.norm.register_forward_hook(lambda m, inp, o: captured.__setitem__("lin_out", inp[0].detach()))

    def values_fwd(indices, scores):
        e = orig_values(indices, scores)
        e.register_hook(lambda gr: captured.__setitem__("d_bag", gr.detach()))
        captured["psw"] = scores.detach()
        return e

    mem.get_indices, mem.values.forward = get_indices, values_fwd
    xd = x.to(device).requires_grad_(True)
    out, idx = mem(xd)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    N = 8 * 2048
    idx_c = idx.cpu().view(N, H * knn)

    # sampled tokens, 8 per sequence at seeded positions (the first and last of each sequence among
    # them): output and input gradient against the float64 oracle at the kernel's selection
    pos = torch.randperm(2048, generator=gen(12))[:6]
    toks = torch.cat([seq * 2048 + torch.cat([torch.tensor([0, 2047]), pos]) for seq in range(8)])
    # the value rows these tokens read, as a compact table with remapped ids (not the 8 GB fp64 table)
    rows, local = torch.unique(idx_c[toks], return_inverse=True)
    P = {nm: p.detach().cpu().double() for nm, p in mem.named_parameters() if nm != "values.weight"}
    P["values.weight"] = mem.values.weight.detach()[rows.to(device)].cpu().double()
    xs = x.view(N, 1, 1024)[toks].double().requires_grad_(True)
    tr = {}
    e_out, _ = pkm_layer.hashing_memory_forward(xs, P, H, knn, idx=idx_c[toks].view(-1, knn),
                                                bag_idx=local.view(-1, knn), trace=tr)
    for t in tr.values():
        t.retain_grad()
    e_out.backward(dout.view(N, 1, 1024)[toks].double())
    out_c = out.detach().cpu().view(N, 1024)
    # out = h @ Wv^T + bv: each element within 2e-2 of the sum of its terms' magnitudes (the
    # rounding bound of a sum with cancellation; a bf16 h carries 2^-9 relative rounding per term)
    Wv, bv = P["value_proj.weight"], P["value_proj.bias"]
    c_out = tr["h"].detach().abs() @ Wv.abs().t() + bv.abs()
    assert_rel_close(out_c[toks], e_out.view(-1, 1024), 2e-2, "sampled out", cond=c_out)
    # dx = d(q_lin) @ Wq + d(s) @ Ws: the same bound
    Wq, Ws = P["query_proj.query_mlps.0.weight"], P["swilu_projection.weight"]
    c_dx = tr["q_lin"].grad.abs() @ Wq.abs() + tr["s"].grad.abs() @ Ws.abs()
    dx_c = xd.grad.cpu().view(N, 1024)[toks]
    assert_rel_close(dx_c, xs.grad.view(-1, 1024), 2e-2, "sampled dx", cond=c_dx)

    # retrieval of the sampled tokens: bit-exact from the kernel's own sub-scores
    qs = captured["query"].view(N, H, 512)[toks.to(device)]
    sc, ix, i1, i2, s1, s2 = [t.cpu() for t in score_topk(qs, mem.keys.detach(), H, knn, "dot", True)]
    e_sc, e_ix, _, _ = ref.select(s1, s2, knn)
    assert torch.equal(ix.view(-1, H, knn), e_ix) and torch.equal(ix.view(-1, H * knn), idx_c[toks])

    # sampled rows of the value gradient: sum over their lookups of psw * d_bag (float64)
    psw = captured["psw"].cpu().double().view(N, H * knn)
    d_bag = captured["d_bag"].cpu().double()
    gW = mem.values.weight.grad
    # 64 rows: the 8 most looked-up ones and 56 at seeded lookup positions
    counts = torch.bincount(idx_c.view(-1), minlength=n * n)
    hot = torch.topk(counts, 8).indices
    some = idx_c.view(-1)[torch.randperm(idx_c.numel(), generator=gen(13))[:56]]
    for r in torch.cat([hot, some]).tolist():
        bags, slots = (idx_c == r).nonzero(as_tuple=True)
        e = (psw[bags, slots, None] * d_bag[bags]).sum(0)
        c = (psw[bags, slots, None].abs() * d_bag[bags].abs()).sum(0)
        assert_rel_close(gW[r].cpu(), e, 2e-2, f"value grad row {r} ({len(bags)} lookups)", cond=c)
    untouched = torch.ones(n * n, dtype=torch.bool)
    untouched[idx_c.view(-1)] = False
    rows = untouched.nonzero().view(-1)[:1000]
    assert (gW[rows.to(device)] == 0).all()

    # keys and query weight: float32 torch products of the dense sub-score gradient
    d_sc = captured["d_scores"].float().view(N, H, knn)
    ids = idx.detach().view(N, H, knn)
    dS = torch.zeros((H, 2, N, n), dtype=torch.float32, device=device)
    for c, ic in ((0, ids // n), (1, ids % n)):
        dS[:, c].scatter_add_(2, ic.permute(1, 0, 2), d_sc.permute(1, 0, 2))
    q = captured["query"].float().view(N, H, 2, 256).permute(1, 2, 0, 3).reshape(2 * H, N, 256)
    Kh = mem.keys.detach().float().view(2 * H, n, 256)
    D = dS.view(2 * H, N, n)
    # elementwise against the same products over |terms| (the kernels round each dS entry to bf16,
    # as the reference's bf16 autograd does, so a sum with cancellation carries their rounding)
    e_dk = torch.bmm(D.transpose(1, 2), q).reshape(mem.keys.shape)
    c_dk = torch.bmm(D.abs().transpose(1, 2), q.abs()).reshape(mem.keys.shape)
    assert_rel_close(mem.keys.grad, e_dk.cpu(), 2e-2, "d_keys", cond=c_dk.cpu())
    e_dq = torch.bmm(D, Kh).view(H, 2, N, 256).permute(2, 0, 1, 3).reshape(N, H * 512)
    c_dq = torch.bmm(D.abs(), Kh.abs()).view(H, 2, N, 256).permute(2, 0, 1, 3).reshape(N, H * 512)
    assert_rel_close(captured["d_query"].view(N, H * 512), e_dq, 2e-2, "d_query", cond=c_dq)
    # the query Linear's weight gradient: float32 autograd of the RMSNorm on the captured query gradient
    lo = captured["lin_out"].float().requires_grad_(True)
    w = mem.query_proj.norm.weight.detach().float()
    y = w * (lo * torch.rsqrt(lo.pow(2).mean(-1, keepdim=True) + 1e-6))
    y.backward(captured["d_query"].float().view(N, H * 512))
    e_gw = lo.grad.t() @ xd.detach().float().view(N, 1024)
    assert_rel_close(mem.query_proj.query_mlps[0].weight.grad, e_gw, 2e-2, "query weight grad")
