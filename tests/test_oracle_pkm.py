"""Pins of the product-key retrieval oracle (oracle/pkm.py) on the CPU.

Each check is chosen so a plausible mistake fails it: a wrong key-table
layout or query split (known-answer tables), a wrong idw formula (torch.cdist,
a library routine), a wrong tie order (Python sorted on tie-heavy integers),
a wrong cartesian id or rounding (brute force over all n^2 pairs), and the
kernel's pair pruning (equal to the full knn^2 selection, ties included).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pkm as ref
from tests.helpers import gen


def _int_inputs(N, H, n, half, dtype, seed, qlim=1, klim=2):
    g = gen(seed)
    q = torch.randint(-qlim, qlim + 1, (N, H, 2 * half), generator=g).to(dtype)
    k = torch.randint(-klim, klim + 1, (2 * H * n, half), generator=g).to(dtype)
    return q, k


def test_sub_scores_known_answer_layout():
    # key row r = [r, 1]: s_c[t, h, i] = a_c * ((2h + c) * n + i) + b_c
    H, n, half, N = 3, 5, 2, 4
    rows = torch.arange(2 * H * n, dtype=torch.float64)
    keys = torch.stack((rows, torch.ones_like(rows)), 1)
    g = gen(1)
    q = torch.randn((N, H, 2 * half), generator=g, dtype=torch.float64)
    s1, s2 = ref.sub_scores(q, keys, H)
    for t in range(N):
        for h in range(H):
            for c, s in ((0, s1), (1, s2)):
                a, b = q[t, h, 2 * c], q[t, h, 2 * c + 1]
                for i in range(n):
                    assert s[t, h, i].item() == pytest.approx((a * ((2 * h + c) * n + i) + b).item(), rel=1e-12)


def test_sub_scores_idw_matches_cdist():
    H, n, half, N = 2, 16, 8, 6
    g = gen(2)
    q = torch.randn((N, H, 2 * half), generator=g, dtype=torch.float64)
    keys = torch.randn((2 * H * n, half), generator=g, dtype=torch.float64)
    s1, s2 = ref.sub_scores(q, keys, H, ref.IDW)
    Kv = keys.view(H, 2, n, half)
    for c, s in ((0, s1), (1, s2)):
        qc = q[:, :, c * half:(c + 1) * half].permute(1, 0, 2)  # fwpkm.py:863
        d = torch.cdist(qc, Kv[:, c], p=2).permute(1, 0, 2)  # fwpkm.py:864-865
        torch.testing.assert_close(s, -torch.log(1e-3 + d.pow(2)), rtol=1e-10, atol=1e-10)


def test_sub_scores_dot_matches_matmul_and_rounds_once():
    H, n, half, N = 2, 64, 32, 5
    g = gen(3)
    q = torch.randn((N, H, 2 * half), generator=g).to(torch.bfloat16)
    keys = torch.randn((2 * H * n, half), generator=g).to(torch.bfloat16)
    s1, s2 = ref.sub_scores(q, keys, H)
    assert s1.dtype == torch.bfloat16
    Kv = keys.double().view(H, 2, n, half)
    for c, s in ((0, s1), (1, s2)):
        for h in range(H):
            exact = q[:, h, c * half:(c + 1) * half].double() @ Kv[h, c].T
            assert torch.equal(s[:, h], exact.to(torch.bfloat16))


def test_topk_stable_tie_order_bruteforce():
    g = gen(4)
    x = torch.randint(-3, 4, (50, 40), generator=g).float()
    v, i = ref.topk_stable(x, 12)
    for r in range(x.shape[0]):
        want = sorted(range(x.shape[1]), key=lambda j: (-x[r, j].item(), j))[:12]
        assert i[r].tolist() == want
        assert v[r].tolist() == [x[r, j].item() for j in want]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_select_equals_all_pairs_bruteforce_tie_free(dtype):
    H, n, knn, N = 2, 12, 5, 3
    g = gen(5)
    s1 = torch.randn((N, H, n), generator=g, dtype=torch.float64).to(dtype)
    s2 = torch.randn((N, H, n), generator=g, dtype=torch.float64).to(dtype)
    scores, idx, i1, i2 = ref.select(s1, s2, knn)
    for t in range(N):
        for h in range(H):
            bf = ref.brute_force_topk_pairs(s1[t, h], s2[t, h], knn)
            vals = [v for v, _ in bf]
            assert len(set(vals)) == len(vals), "input not tie-free"
            assert idx[t, h].tolist() == [j for _, j in bf]
            assert scores[t, h].tolist() == vals


def test_select_bf16_rounding_bruteforce():
    # bf16 sums are rounded; brute force on tiny n with the same rounding,
    # compared as multisets of values (ids may legitimately differ in ties)
    H, n, knn, N = 1, 10, 6, 8
    g = gen(6)
    s1 = torch.randn((N, H, n), generator=g).to(torch.bfloat16)
    s2 = torch.randn((N, H, n), generator=g).to(torch.bfloat16)
    scores, idx, _, _ = ref.select(s1, s2, knn)
    for t in range(N):
        bf = ref.brute_force_topk_pairs(s1[t, 0], s2[t, 0], knn)
        assert scores[t, 0].float().tolist() == [v for v, _ in bf]
        got = (s1[t, 0].double()[idx[t, 0] // n] + s2[t, 0].double()[idx[t, 0] % n]).float().to(torch.bfloat16)
        assert torch.equal(got, scores[t, 0])


def test_get_indices_matches_numpy_argsort_tie_free():
    H, n, half, knn, N = 2, 32, 16, 8, 7
    g = gen(7)
    q = torch.randn((N, H, 2 * half), generator=g, dtype=torch.float64)
    keys = torch.randn((2 * H * n, half), generator=g, dtype=torch.float64)
    scores, idx, i1, i2, s1, s2 = ref.get_indices(q, keys, H, knn)
    s1n, s2n = s1.numpy(), s2.numpy()
    for t in range(N):
        for h in range(H):
            a1 = np.argsort(-s1n[t, h], kind="stable")[:knn]
            a2 = np.argsort(-s2n[t, h], kind="stable")[:knn]
            assert i1[t, h].tolist() == a1.tolist() and i2[t, h].tolist() == a2.tolist()
            cand = (s1n[t, h][a1][:, None] + s2n[t, h][a2][None, :]).reshape(-1)
            cid = (a1[:, None] * n + a2[None, :]).reshape(-1)
            best = np.argsort(-cand, kind="stable")[:knn]
            assert idx[t, h].tolist() == cid[best].tolist()
            np.testing.assert_array_equal(scores[t, h].numpy(), cand[best])


def test_get_indices_known_answer():
    # keys (h, c, i) = e_0 * (i == target_c(h)) + small distinct noise: the
    # best pair per head is (target_0, target_1), id = target_0 * n + target_1
    H, n, half = 4, 16, 4
    keys = torch.zeros((2 * H * n, half), dtype=torch.float64)
    targets = {}
    for h in range(H):
        for c in range(2):
            tgt = (3 * h + 5 * c + 1) % n
            targets[h, c] = tgt
            for i in range(n):
                keys[ref.key_rows(H, n, c, h, i)] = torch.tensor([1.0 if i == tgt else 0.0, 0.01 * i, 0, 0])
    q = torch.zeros((2, H, 2 * half), dtype=torch.float64)
    q[:, :, 0] = 1.0
    q[:, :, half] = 1.0
    scores, idx, i1, i2, _, _ = ref.get_indices(q, keys, H, 1)
    for h in range(H):
        assert idx[0, h, 0].item() == targets[h, 0] * n + targets[h, 1]
        assert scores[0, h, 0].item() == 2.0


@pytest.mark.parametrize("knn", [1, 2, 5, 16, 32, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pruned_selection_equals_full_with_ties(knn, dtype):
    n = max(64, knn)
    g = gen(100 + knn)
    # small integers: many equal sub-scores and many equal sums
    s1 = torch.randint(-4, 5, (6, 3, n), generator=g).to(dtype)
    s2 = torch.randint(-4, 5, (6, 3, n), generator=g).to(dtype)
    full = ref.select(s1, s2, knn)
    pruned = ref.select_pruned(s1, s2, knn)
    for a, b in zip(full, pruned):
        assert torch.equal(a, b)
    # and on continuous values with bf16/f32 rounding
    s1 = torch.randn((6, 3, n), generator=g).to(dtype)
    s2 = torch.randn((6, 3, n), generator=g).to(dtype)
    for a, b in zip(ref.select(s1, s2, knn), ref.select_pruned(s1, s2, knn)):
        assert torch.equal(a, b)


def test_pruned_pair_counts():
    # candidates per (token, head): 50 / 119 / 280 for knn 16 / 32 / 64
    for knn, want in ((16, 50), (32, 119), (64, 280)):
        assert sum(knn // (a + 1) for a in range(knn)) == want


def test_integer_inputs_are_exact_in_bf16():
    # the GPU parity test relies on integer inputs whose sub-scores are exact
    # integers (|s| <= 2 * half) before the one rounding to bf16
    q, k = _int_inputs(4, 2, 64, 256, torch.bfloat16, 8)
    s1, _ = ref.sub_scores(q, k, 2, out_dtype=torch.float64)
    assert torch.equal(s1, s1.round()) and s1.abs().max() <= 2 * 256


def test_score_grad_dense_matches_autograd():
    """The dense sub-score gradient is what autograd gives through
    s1.gather + s2.gather (duplicate sub-keys included), float64."""
    N, H, n, knn = 7, 3, 40, 9
    g = gen(9)
    s1 = torch.randn((N, H, n), generator=g, dtype=torch.float64, requires_grad=True)
    s2 = torch.randn((N, H, n), generator=g, dtype=torch.float64, requires_grad=True)
    _, idx, _, _ = ref.select(s1.detach(), s2.detach(), knn)
    d = torch.randn((N, H, knn), generator=g, dtype=torch.float64)
    ds1 = torch.randn((N, H, n), generator=g, dtype=torch.float64)
    ds2 = torch.randn((N, H, n), generator=g, dtype=torch.float64)
    sel = s1.gather(2, idx // n) + s2.gather(2, idx % n)
    ((sel * d).sum() + (s1 * ds1).sum() + (s2 * ds2).sum()).backward()
    got = ref.score_grad_dense(idx, d, n, ds1, ds2).double()
    torch.testing.assert_close(got[:, 0].permute(1, 0, 2), s1.grad, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(got[:, 1].permute(1, 0, 2), s2.grad, rtol=1e-6, atol=1e-6)
    # duplicates really occur: some sub-key is shared by several selected pairs
    assert any(len(set((idx[t, h] // n).tolist())) < knn for t in range(N) for h in range(H))
