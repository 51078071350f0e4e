"""Product-key selection bit-exact against the reference's own op sequence on
tie-free seeded inputs (GPU).

torch.topk leaves the order of equal scores unspecified, so the reference's
selection is defined only where no ties reach the boundary or the order of
the selected entries. Two input families make it defined, and the kernel's
indices and scores are compared with the oracle's restatement of the
reference's einsum / topk / cartesian / topk / gather sequence
(oracle.pkm_layer.get_indices_torch, pkm/memory.py:250-289) evaluated on the
oracle's own sub-scores (not the kernel's):

  * float32, margin-certified: random normal queries and keys; every
    (token, head) row whose per-half top-(k+1) or cartesian top-(k+1) scores
    (computed in float64) have two neighbours closer than 1e-4 of the row's
    score scale is redrawn, so the float32 rounding of any implementation
    cannot reorder them;
  * bfloat16, exact: one-hot queries (a single 1.0 per half) against keys
    whose entries are bf16 values, so every dot product is exact in float32
    in any summation order; each key column holds 33 distinct top values
    8x (x = -1..31) in half 0 and 0..7 then 25 values in [-612, -516] in
    half 1, the rest far below: the per-half top-33 are distinct, and the
    cartesian sums 8x + y of the top pairs are distinct integers below 256,
    exact in bf16, so the top-33 candidates are distinct after rounding too.

At the layer's head shape (8 heads, 1024 keys per half, k_dim 512, knn 32)
and at the CPU parity configuration's (4 heads, 256 keys per half, k_dim 512,
knn 32).
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd.product_keys import score_topk
from oracle import pkm as ref
from oracle import pkm_layer
from tests.helpers import assert_rel_close, gen

pytestmark = pytest.mark.gpu

SHAPES = {"layer": (8, 1024, 256, 32), "cpu_parity_config": (4, 256, 256, 32)}
MARGIN = 1e-4


def _row_gaps(s1, s2, knn):
    """Smallest gap between neighbours among each row's per-half top-(k+1)
    and cartesian top-(k+1) sums, over the row's score scale. s: [N, H, n]."""
    out = []
    tops = []
    for s in (s1, s2):
        v = s.sort(dim=-1, descending=True).values[..., : knn + 1]
        out.append((v[..., :-1] - v[..., 1:]).min(-1).values)
        tops.append(v)
    cand = (tops[0][..., :, None] + tops[1][..., None, :]).flatten(-2).sort(dim=-1, descending=True).values
    cand = cand[..., : knn + 1]
    out.append((cand[..., :-1] - cand[..., 1:]).min(-1).values)
    scale = torch.maximum(s1.abs().amax(-1), s2.abs().amax(-1))
    return torch.stack(out).min(0).values / scale


def _certified_fp32(N, H, n, half, knn, seed):
    g = gen(seed)
    q = torch.randn((N, H, 2 * half), generator=g)
    k = (torch.rand((2 * H * n, half), generator=g) * 2 - 1) * half**-0.5
    for _ in range(200):
        s1, s2 = ref.sub_scores(q, k, H, out_dtype=torch.float64)
        bad = _row_gaps(s1, s2, knn) < MARGIN  # [N, H]
        if not bad.any():
            return q, k
        rows = bad.nonzero()
        q[rows[:, 0], rows[:, 1]] = torch.randn((rows.shape[0], 2 * half), generator=g)
    raise RuntimeError("could not certify every row")


def _exact_bf16(N, H, n, half, knn, seed):
    assert knn == 32 and half >= 2
    g = gen(seed)
    K = torch.full((H, 2, n, half), -2048.0)
    for h in range(H):
        for d in range(half):
            perm = torch.randperm(n, generator=g)
            K[h, 0, perm[:33], d] = 8.0 * torch.arange(31, -2, -1, dtype=torch.float32)
            K[h, 1, perm[:8], d] = torch.arange(7, -1, -1, dtype=torch.float32)
            K[h, 1, perm[8:33], d] = -(516.0 + 4.0 * torch.arange(25, dtype=torch.float32))
    q = torch.zeros((N, H, 2, half))
    cols = torch.randint(0, half, (N, H, 2), generator=g)
    q.scatter_(3, cols[..., None], 1.0)
    return q.reshape(N, H, 2 * half).to(torch.bfloat16), K.reshape(2 * H * n, half).to(torch.bfloat16)


def _check(q, k, H, knn, device, tol):
    N = q.shape[0]
    scores, idx, i1, i2, s1, s2 = [t.cpu() for t in score_topk(q.to(device), k.to(device), H, knn, "dot", True)]
    e1, e2 = ref.sub_scores(q, k, H)  # float64, rounded once to the input dtype
    assert_rel_close(s1, e1, tol, "s1")
    assert_rel_close(s2, e2, tol, "s2")
    # the reference's own op sequence on the oracle's scores
    r_scores, r_idx = pkm_layer.get_indices_torch(q.reshape(N * H, -1), k, H, knn)
    assert torch.equal(idx, r_idx), "indices differ from the reference op sequence"
    assert_rel_close(scores, r_scores, tol, "selected scores")
    # and the per-half selections
    v1, j1 = ref.topk_stable(e1, knn)
    v2, j2 = ref.topk_stable(e2, knn)
    assert torch.equal(i1, j1) and torch.equal(i2, j2)


@pytest.mark.parametrize("name", list(SHAPES))
def test_fp32_margin_certified(name, device):
    H, n, half, knn = SHAPES[name]
    q, k = _certified_fp32(256, H, n, half, knn, seed=81 + n)
    _check(q, k, H, knn, device, 1e-5)


@pytest.mark.parametrize("name", list(SHAPES))
def test_bf16_exact_dot_products(name, device):
    H, n, half, knn = SHAPES[name]
    q, k = _exact_bf16(512, H, n, half, knn, seed=91 + n)
    s1, s2 = ref.sub_scores(q, k, H, out_dtype=torch.float64)
    assert (_row_gaps(s1, s2, knn) > 0).all()  # tie-free by construction
    N = q.shape[0]
    scores, idx, *_ = [t.cpu() for t in score_topk(q.to(device), k.to(device), H, knn, "dot", True)]
    r_scores, r_idx = pkm_layer.get_indices_torch(q.reshape(N * H, -1), k, H, knn)
    assert torch.equal(idx, r_idx) and torch.equal(scores, r_scores)
    _check(q, k, H, knn, device, 0.0)
