"""The streaming scoring kernel against the oracle (GPU).

pkm_score_topk sends bfloat16 dot scores with knn <= 32 and a half key dim
of 128 or 256 (the layer's configuration) to its streaming kernel, which keeps
a sorted running top-32 per token in registers and appends the scores that
can reach it to LDS slots, merging 32 at a time. The cases aim at its own
paths: workgroup and wave tails (token counts that are not multiples of 256
or 64), head counts whose 2H does not divide the 8 XCDs, every knn up to 32,
the largest n_keys, all-equal scores (a zero query: index order), key orders
in which every score beats all earlier ones (every tile appends all of its
scores, so the wave merges after every tile) or none does, +0 / -0 ties, and
many tokens at the layer's shape.
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd.product_keys import score_topk
from oracle import pkm as ref
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu

# (tokens, heads, n_keys, half, knn)
INT_SHAPES = [
    (1, 1, 64, 128, 1),
    (63, 3, 192, 128, 7),
    (257, 2, 2048, 128, 32),
    (300, 8, 1024, 256, 32),
    (65, 5, 512, 256, 16),
    (129, 4, 256, 256, 31),
]


def _ids(shape):
    return "N{}-H{}-n{}-h{}-k{}".format(*shape)


def _run(q, k, H, knn, device):
    out = score_topk(q.to(device), k.to(device), H, knn, "dot", sub_outputs=True)
    torch.cuda.synchronize()
    return [t.cpu() for t in out]


def _check_exact(q, k, H, knn, device):
    N = q.shape[0]
    scores, idx, i1, i2, s1, s2 = _run(q, k, H, knn, device)
    e_scores, e_idx, e_i1, e_i2, e_s1, e_s2 = ref.get_indices(q, k, H, knn)
    assert torch.equal(s1, e_s1) and torch.equal(s2, e_s2)
    assert torch.equal(i1, e_i1) and torch.equal(i2, e_i2)
    assert torch.equal(idx.view(N, H, knn), e_idx)
    assert torch.equal(scores.view(N, H, knn), e_scores)
    # without the sub-score outputs: the same selection
    two = score_topk(q.to(device), k.to(device), H, knn, "dot")
    assert torch.equal(two[0].cpu(), scores) and torch.equal(two[1].cpu(), idx)
    return i1


@pytest.mark.parametrize("shape", INT_SHAPES, ids=_ids)
def test_integer_inputs_bit_exact(device, shape):
    N, H, n, half, knn = shape
    g = gen(31)
    q = torch.randint(-1, 2, (N, H, 2 * half), generator=g).to(torch.bfloat16)
    k = torch.randint(-2, 3, (2 * H * n, half), generator=g).to(torch.bfloat16)
    _check_exact(q, k, H, knn, device)


@pytest.mark.parametrize("knn", list(range(1, 33)))
def test_every_knn(device, knn):
    N, H, n, half = 70, 2, 320, 128
    g = gen(100 + knn)
    q = torch.randint(-1, 2, (N, H, 2 * half), generator=g).to(torch.bfloat16)
    k = torch.randint(-2, 3, (2 * H * n, half), generator=g).to(torch.bfloat16)
    _check_exact(q, k, H, knn, device)


@pytest.mark.parametrize("shape", [(1000, 8, 1024, 256, 32), (517, 4, 512, 128, 16)], ids=_ids)
def test_random_inputs(device, shape):
    N, H, n, half, knn = shape
    g = gen(37)
    q = torch.randn((N, H, 2 * half), generator=g).to(torch.bfloat16)
    k = ((torch.rand((2 * H * n, half), generator=g) * 2 - 1) * half**-0.5).to(torch.bfloat16)
    scores, idx, i1, i2, s1, s2 = _run(q, k, H, knn, device)
    e_s1, e_s2 = ref.sub_scores(q, k, H)
    assert_rel_close(s1, e_s1, REL_TOL[torch.bfloat16], "s1")
    assert_rel_close(s2, e_s2, REL_TOL[torch.bfloat16], "s2")
    # the selection is a function of the rounded sub-scores: bit-exact
    e_scores, e_idx, e_i1, e_i2 = ref.select(s1, s2, knn)
    assert torch.equal(i1, e_i1) and torch.equal(i2, e_i2)
    assert torch.equal(idx.view(N, H, knn), e_idx)
    assert torch.equal(scores.view(N, H, knn), e_scores)


def test_zero_query_index_order(device):
    """Every score equal: the lists are the index order."""
    N, H, n, half, knn = 80, 2, 1024, 256, 32
    g = gen(41)
    q = torch.zeros((N, H, 2 * half), dtype=torch.bfloat16)
    k = torch.randn((2 * H * n, half), generator=g).to(torch.bfloat16)
    i1 = _check_exact(q, k, H, knn, device)
    assert torch.equal(i1[0, 0], torch.arange(knn))


def _one_hot_keys(N, H, n, half, col_values, seed):
    """One-hot queries (a single 1.0 per half, in column `col`) against keys
    whose column `col` holds col_values[i] for key i: every score is that
    bf16 value, exactly."""
    g = gen(seed)
    cols = torch.randint(0, half, (N, H, 2), generator=g)
    q = torch.zeros((N, H, 2, half))
    q.scatter_(3, cols[..., None], 1.0)
    K = torch.randn((H, 2, n, half), generator=g)
    for h in range(H):
        for c in range(2):
            for col in cols[:, h, c].unique().tolist():
                K[h, c, :, col] = col_values
    return q.reshape(N, H, 2 * half).to(torch.bfloat16), K.reshape(2 * H * n, half).to(torch.bfloat16)


@pytest.mark.parametrize("order", ["increasing", "decreasing", "increasing_negative"])
def test_monotone_key_orders(device, order):
    """Increasing: every tile beats everything before it (all its scores are
    appended and merged); decreasing: nothing after the first tiles passes.
    The bf16 values repeat in runs (i / 16 rounded), so ties cross tiles."""
    N, H, n, half, knn = 96, 2, 1024, 256, 32
    v = (torch.arange(n, dtype=torch.float32) + 1) / 16
    vals = {"increasing": v, "decreasing": v.flip(0), "increasing_negative": -v.flip(0)}[order]
    q, k = _one_hot_keys(N, H, n, half, vals, seed=43)
    _check_exact(q, k, H, knn, device)


def test_signed_zero_ties(device):
    """+0 and -0 scores are equal values: after the positive ones, the zeros
    come in index order whatever their sign."""
    N, H, n, half, knn = 64, 2, 256, 128, 32
    vals = torch.zeros(n)
    vals[1::2] = -0.0
    vals[torch.tensor([5, 77, 130, 200, 201, 255])] = 1.0
    vals[torch.tensor([3, 9, 100])] = -1.0
    q, k = _one_hot_keys(N, H, n, half, vals, seed=47)
    i1 = _check_exact(q, k, H, knn, device)
    zeros = [i for i in range(n) if vals[i] == 0][: knn - 6]
    assert i1[0, 0].tolist() == [5, 77, 130, 200, 201, 255] + zeros


@pytest.mark.parametrize("which", [1, 2])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_single_sub_score_output_through_c_abi(device, which, dtype):
    """One sub-score pointer NULL, the other given, straight through the C ABI
    (the streaming kernel for bf16, the tile kernel for float32): the given
    half equals the full call's and the call does not touch the NULL one."""
    from modelos_amd import _lib

    N, H, n, half, knn = 300, 4, 512, 128, 32
    g = gen(77 + which)
    q = torch.randn((N, H, 2 * half), generator=g).to(dtype).to(device)
    k = torch.randn((2 * H * n, half), generator=g).to(dtype).to(device)
    full = score_topk(q, k, H, knn, "dot", sub_outputs=True)
    scores = torch.empty((N * H, knn), dtype=dtype, device=device)
    idx = torch.empty((N * H, knn), dtype=torch.long, device=device)
    s_out = torch.empty((N, H, n), dtype=dtype, device=device)
    s1, s2 = (s_out, None) if which == 1 else (None, s_out)
    _lib.call(
        "pkm_score_topk",
        _lib.ptr(q), _lib.ptr(k), N, H, n, half, knn, _lib.SCORE_CODES["dot"], _lib.dtype_code(q),
        _lib.ptr(scores), _lib.ptr(idx), None, None, _lib.ptr(s1), _lib.ptr(s2), _lib.stream_of(q.device),
    )
    torch.cuda.synchronize()
    assert torch.equal(idx, full[1]) and torch.equal(scores, full[0])
    assert torch.equal(s_out, full[4] if which == 1 else full[5])
