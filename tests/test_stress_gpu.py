"""Large-memory stress shape on the GPU: 16 heads, 2048 keys per half
(4,194,304 value slots), k_dim 512, knn 64, value dim 2048 (a 16 GiB bf16
table), 4 x 4096 tokens, with sub-key scores skewed towards low sub-key ids
(a Zipf(1.1) pre-bias) so that a few value rows collect thousands of lookups
(the backward's heavy-row path at full size).

Checked:
- retrieval: sampled tokens against the oracle (sub-scores within the bf16
  tolerance, selection bit-exact from the kernel's sub-scores) and, over every
  row, best-first order, ids in range and distinct;
- value bag: sampled bags of the forward against the oracle; the backward is
  bitwise deterministic, rows never looked up are exactly zero, the column sum
  of the table gradient equals sum_b (sum_j psw[b, j]) g[b], and sampled rows
  (the hottest ones included) and sampled psw-gradients match float32
  references.
"""
import pytest
import torch

from oracle import pkm as ref
from oracle import eb as eref
from tests.helpers import REL_TOL, assert_rel_close

pytestmark = pytest.mark.gpu

N_TOK, H, N_KEYS, HALF, KNN, V_DIM = 4 * 4096, 16, 2048, 256, 64, 2048


@pytest.fixture(scope="module")
def stress(device):
    """(query, keys, scores, ids, sub-scores) at the stress shape."""
    from modelos_amd.product_keys import score_topk

    gd = torch.Generator(device=device).manual_seed(51)
    q = torch.randn((N_TOK, H, 2 * HALF), generator=gd, device=device)
    k = (torch.rand((2 * H * N_KEYS, HALF), generator=gd, device=device) * 2 - 1) * HALF**-0.5
    # Zipf pre-bias: element 0 of each query half is 1, element 0 of sub-key i
    # is 1.5 / (i + 1)^1.1, so low sub-key ids score higher
    q[:, :, 0] = 1.0
    q[:, :, HALF] = 1.0
    i = torch.arange(N_KEYS, device=device, dtype=torch.float32)
    k.view(2 * H, N_KEYS, HALF)[:, :, 0] = 1.5 / (i + 1.0) ** 1.1
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    scores, ids, _, _, s1, s2 = score_topk(q, k, H, KNN, "dot", sub_outputs=True)
    torch.cuda.synchronize()
    return q, k, scores, ids, s1, s2


def test_stress_retrieval(stress):
    q, k, scores, ids, s1, s2 = stress
    dev = q.device
    rows = torch.randint(0, N_TOK, (48,), generator=torch.Generator().manual_seed(52))
    e_s1, e_s2 = ref.sub_scores(q[rows.to(dev)].cpu(), k.cpu(), H)
    assert_rel_close(s1[rows.to(dev)].cpu(), e_s1, REL_TOL[torch.bfloat16], "s1")
    assert_rel_close(s2[rows.to(dev)].cpu(), e_s2, REL_TOL[torch.bfloat16], "s2")
    e_scores, e_ids, _, _ = ref.select(s1[rows.to(dev)].cpu(), s2[rows.to(dev)].cpu(), KNN)
    assert torch.equal(ids.view(N_TOK, H, KNN)[rows.to(dev)].cpu(), e_ids)
    assert torch.equal(scores.view(N_TOK, H, KNN)[rows.to(dev)].cpu(), e_scores)
    sc = scores.float()
    assert bool((sc[:, :-1] >= sc[:, 1:]).all())
    assert int(ids.min()) >= 0 and int(ids.max()) < N_KEYS * N_KEYS
    srt = ids.sort(dim=1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all())


def test_stress_value_bag(stress):
    from modelos_amd import embedding_bag as eb

    _, _, scores, ids, _, _ = stress
    dev = ids.device
    K, D = N_KEYS * N_KEYS, V_DIM
    idx = ids.view(N_TOK, H * KNN)
    psw = torch.softmax(scores.float().view(N_TOK, H, KNN), -1).to(torch.bfloat16).view(N_TOK, H * KNN)
    counts = torch.bincount(idx.reshape(-1), minlength=K)
    assert int(counts.max()) > 256, "the skew must produce heavy rows"

    gd = torch.Generator(device=dev).manual_seed(53)
    W = (torch.randn((K, D), generator=gd, device=dev, dtype=torch.bfloat16) * 0.02)
    g = torch.randn((N_TOK, D), generator=gd, device=dev, dtype=torch.bfloat16)

    out = eb.eb_forward(idx, W, psw)
    bags = torch.randint(0, N_TOK, (32,), generator=torch.Generator().manual_seed(54)).to(dev)
    bi, bp = idx[bags].cpu(), psw[bags].cpu()
    local = torch.arange(bi.numel()).view(bi.shape)
    assert_rel_close(out[bags], eref.eb_forward(local, W[bi.reshape(-1)].cpu(), bp), 2e-2, "forward (sampled bags)")
    del out

    gW, gp = eb.eb_backward(idx, W, psw, g)
    gW2, gp2 = eb.eb_backward(idx, W, psw, g)
    assert torch.equal(gW, gW2) and torch.equal(gp, gp2), "backward is not bitwise deterministic"
    del gW2, gp2
    # per row chunk (no float32 copy of the whole table): untouched rows are
    # zero, and the column sums
    colsum = torch.zeros(D, device=dev)
    for c0 in range(0, K, 1 << 19):
        blk = gW[c0:c0 + (1 << 19)]
        assert not bool(blk[counts[c0:c0 + (1 << 19)] == 0].any()), "a row never looked up is not zero"
        colsum += blk.float().sum(0)
        del blk
    expect = (psw.float().sum(1, keepdim=True) * g.float()).sum(0)
    assert_rel_close(colsum, expect, 2e-2, "column-sum checksum")

    # sampled rows: the 8 hottest and 120 random touched ones, against a
    # float32 index_add restricted to them
    touched = (counts > 0).nonzero().squeeze(1)
    pick = torch.randperm(touched.numel(), generator=torch.Generator().manual_seed(55))[:120].to(dev)
    rows = torch.unique(torch.cat([counts.topk(8).indices, touched[pick]]))
    slot = torch.full((K,), -1, dtype=torch.long, device=dev)
    slot[rows] = torch.arange(rows.numel(), device=dev)
    flat = idx.reshape(-1)
    hit = (slot[flat] >= 0).nonzero().squeeze(1)
    contrib = psw.reshape(-1)[hit].float()[:, None] * g[hit // idx.shape[1]].float()
    exp_rows = torch.zeros((rows.numel(), D), device=dev).index_add_(0, slot[flat[hit]], contrib)
    assert_rel_close(gW[rows], exp_rows, 2e-2, "sampled grad_weight rows (hot rows included)")

    e_gp = (W[idx[bags]].float() * g[bags].float()[:, None, :]).sum(-1)
    assert_rel_close(gp[bags], e_gp, 2e-2, "sampled grad_psw")
