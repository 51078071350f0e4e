"""GPU parity of product-key retrieval (pkm_score_topk) against the oracle.

Three levels:
  * integer inputs (exact sub-scores, many ties): every output bit-exact
    against oracle.pkm.get_indices, tie order included;
  * random inputs: sub-scores within the dtype's tolerance of the float64
    oracle, and the selection (per-half top-k, cartesian top-k, ids) bit-exact
    against oracle.pkm.select applied to the kernel's own sub-scores;
  * gradients of the autograd wrapper against float64 autograd of the
    oracle's scores at the kernel's selection.
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd import _lib
from modelos_amd.product_keys import product_key_topk, score_grad_dense, score_topk
from oracle import pkm as ref
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu

# (tokens, heads, n_keys, half, knn)
SHAPES = [
    (70, 8, 1024, 256, 32),  # PKM layer head shape (k_dim 512, 1024^2 slots)
    (37, 4, 512, 128, 16),  # fast-weight PKM (k_dim 256, 512^2 slots)
    (20, 16, 2048, 256, 64),  # 4M-slot table, knn 64 (16-token tiles)
    (5, 2, 64, 32, 64),  # knn == n_keys
    (3, 1, 64, 32, 1),  # knn 1
    (33, 3, 192, 64, 7),  # odd knn
    (24, 2, 1024, 64, 64),  # knn 64 on 1024 keys: 65-128 threshold candidates per row
]
# shapes outside the tuned kernels' limits (the generic kernel)
GENERIC_SHAPES = [
    (21, 3, 100, 10, 7),  # n_keys not a multiple of 64, half not a multiple of 16
    (9, 2, 1000, 256, 32),  # n_keys 1000
    (6, 2, 512, 64, 128),  # knn 128
    (4, 2, 4096, 128, 64),  # n_keys above 2048
    (5, 1, 16, 8, 16),  # knn == n_keys, tiny
    (3, 1, 1, 4, 1),  # a single sub-key
    (7, 2, 64, 33, 5),  # half 33
    (2, 1, 700, 16, 700),  # knn == n_keys, 700
]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
DTYPE_IDS = ["f32", "bf16", "f16"]


def _ids(shape):
    return "N{}-H{}-n{}-h{}-k{}".format(*shape)


def _random_inputs(N, H, n, half, dtype, seed):
    g = gen(seed)
    q = torch.randn((N, H, 2 * half), generator=g).to(dtype)
    k = (torch.rand((2 * H * n, half), generator=g) * 2 - 1).mul(half**-0.5).to(dtype)
    return q, k


def _int_inputs(N, H, n, half, dtype, seed):
    g = gen(seed)
    q = torch.randint(-1, 2, (N, H, 2 * half), generator=g).to(dtype)
    k = torch.randint(-2, 3, (2 * H * n, half), generator=g).to(dtype)
    return q, k


def _run(q, k, H, knn, score_type, device):
    out = score_topk(q.to(device), k.to(device), H, knn, score_type, sub_outputs=True)
    torch.cuda.synchronize()
    return [t.cpu() for t in out]


@pytest.mark.parametrize("shape", SHAPES + GENERIC_SHAPES, ids=_ids)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_integer_inputs_bit_exact(device, shape, dtype):
    N, H, n, half, knn = shape
    q, k = _int_inputs(N, H, n, half, dtype, seed=11)
    scores, idx, i1, i2, s1, s2 = _run(q, k, H, knn, "dot", device)
    e_scores, e_idx, e_i1, e_i2, e_s1, e_s2 = ref.get_indices(q, k, H, knn)
    assert torch.equal(s1, e_s1) and torch.equal(s2, e_s2)
    assert torch.equal(i1, e_i1) and torch.equal(i2, e_i2)
    assert torch.equal(idx.view(N, H, knn), e_idx)
    assert torch.equal(scores.view(N, H, knn), e_scores)


@pytest.mark.parametrize("shape", SHAPES + GENERIC_SHAPES, ids=_ids)
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("score_type", ["dot", "idw"])
def test_random_inputs(device, shape, dtype, score_type):
    N, H, n, half, knn = shape
    q, k = _random_inputs(N, H, n, half, dtype, seed=12)
    scores, idx, i1, i2, s1, s2 = _run(q, k, H, knn, score_type, device)
    e_s1, e_s2 = ref.sub_scores(q, k, H, score_type)
    assert_rel_close(s1, e_s1, REL_TOL[dtype], "s1")
    assert_rel_close(s2, e_s2, REL_TOL[dtype], "s2")
    # the selection is a function of the rounded sub-scores: bit-exact
    e_scores, e_idx, e_i1, e_i2 = ref.select(s1, s2, knn)
    assert torch.equal(i1, e_i1) and torch.equal(i2, e_i2)
    assert torch.equal(idx.view(N, H, knn), e_idx)
    assert torch.equal(scores.view(N, H, knn), e_scores)


@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_all_scores_equal(device, dtype):
    """A zero query makes every score equal: the order is the index order
    (per half 0..knn-1, then the cartesian flat positions)."""
    N, H, n, half, knn = 9, 2, 256, 64, 16
    q = torch.zeros((N, H, 2 * half), dtype=dtype)
    _, k = _random_inputs(N, H, n, half, dtype, seed=19)
    scores, idx, i1, i2, s1, s2 = _run(q, k, H, knn, "dot", device)
    e_scores, e_idx, e_i1, e_i2, e_s1, e_s2 = ref.get_indices(q, k, H, knn)
    assert torch.equal(i1, e_i1) and torch.equal(i2, e_i2)
    assert torch.equal(idx.view(N, H, knn), e_idx) and torch.equal(scores.view(N, H, knn), e_scores)
    assert torch.equal(i1[0, 0], torch.arange(knn))


def test_sub_outputs_optional_and_query_views(device):
    N, H, n, half, knn = 40, 4, 256, 64, 8
    q, k = _random_inputs(N, H, n, half, torch.bfloat16, seed=13)
    qd, kd = q.to(device), k.to(device)
    full = score_topk(qd, kd, H, knn, "dot", sub_outputs=True)
    two = score_topk(qd.view(N * H, 2 * half), kd, H, knn, "dot")
    assert len(two) == 2
    assert torch.equal(full[0], two[0]) and torch.equal(full[1], two[1])


def test_deterministic(device):
    N, H, n, half, knn = 64, 8, 1024, 256, 32
    q, k = _random_inputs(N, H, n, half, torch.bfloat16, seed=14)
    a = score_topk(q.to(device), k.to(device), H, knn)
    b = score_topk(q.to(device), k.to(device), H, knn)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_empty_tokens(device):
    q = torch.empty((0, 4, 64), dtype=torch.bfloat16, device=device)
    k = torch.randn((2 * 4 * 64, 32), device=device).to(torch.bfloat16)
    scores, idx = score_topk(q, k, 4, 8)
    assert scores.shape == (0, 8) and idx.shape == (0, 8)


@pytest.mark.parametrize(
    "case",
    [
        dict(n=64, knn=65, half=32, dtype=torch.float32, err=ValueError),  # knn > n_keys
        dict(n=2048, knn=1025, half=8, dtype=torch.float32, err=_lib.PkmError),  # knn > 1024
        dict(n=16385, knn=4, half=4, dtype=torch.float32, err=_lib.PkmError),  # n_keys > 16384
        dict(n=64, knn=4, half=32, dtype=torch.float64, err=TypeError),  # dtype
    ],
)
def test_unsupported_sizes_raise(device, case):
    H = 2
    q = torch.randn((3, H, 2 * case["half"]), device=device).to(case["dtype"])
    k = torch.randn((2 * H * case["n"], case["half"]), device=device).to(case["dtype"])
    with pytest.raises(case["err"]):
        score_topk(q, k, H, case["knn"])


def _reference_grads(q, k, H, knn, score_type, idx, d_scores, d_s1=None, d_s2=None):
    """float64 autograd of the oracle's scores at the kernel's selection:
    scores = s1[id // n] + s2[id % n] (memory.py:274-285 with the gather
    fixed), plus optional upstream gradients of the full sub-scores."""
    q64 = q.double().requires_grad_(True)
    k64 = k.double().requires_grad_(True)
    N = q.shape[0]
    n = k.shape[0] // (2 * H)
    s1, s2 = ref.sub_scores(q64, k64, H, score_type, out_dtype=torch.float64)
    ids = idx.view(N, H, knn)
    sel = s1.gather(2, ids // n) + s2.gather(2, ids % n)
    loss = (sel * d_scores.view(N, H, knn).double()).sum()
    if d_s1 is not None:
        loss = loss + (s1 * d_s1.double()).sum() + (s2 * d_s2.double()).sum()
    loss.backward()
    return q64.grad, k64.grad


@pytest.mark.parametrize("score_type", ["dot", "idw"])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
@pytest.mark.parametrize("sub", [False, True], ids=["topk", "topk+sub"])
@pytest.mark.parametrize("shape", [(45, 4, 256, 64, 16), (13, 3, 300, 24, 80)], ids=["tuned", "generic"])
def test_gradients(device, score_type, dtype, sub, shape):
    N, H, n, half, knn = shape
    q, k = _random_inputs(N, H, n, half, dtype, seed=15)
    g = gen(16)
    d_scores = torch.randn((N * H, knn), generator=g).to(dtype)
    d_s1 = torch.randn((N, H, n), generator=g).to(dtype) if sub else None
    d_s2 = torch.randn((N, H, n), generator=g).to(dtype) if sub else None
    qd = q.to(device).requires_grad_(True)
    kd = k.to(device).requires_grad_(True)
    outs = product_key_topk(qd, kd, H, knn, score_type, sub_outputs=sub)
    loss = (outs[0].float() * d_scores.to(device).float()).sum()
    if sub:
        loss = loss + (outs[4].float() * d_s1.to(device).float()).sum() + (outs[5].float() * d_s2.to(device).float()).sum()
    loss.backward()
    e_dq, e_dk = _reference_grads(q, k, H, knn, score_type, outs[1].cpu(), d_scores, d_s1, d_s2)
    # float16 (no tolerance stated for it): 10 units of its rounding, as the sums over tokens carry the
    # rounding of every fp16 sub-score gradient
    tol = REL_TOL[dtype] if dtype != torch.float16 else 5e-3
    assert_rel_close(qd.grad.cpu(), e_dq, tol, "d_query")
    assert_rel_close(kd.grad.cpu(), e_dk, tol, "d_keys")


def test_full_size_layer_shape_sampled(device):
    """16384 tokens x 8 heads, 1024 keys per half, k_dim 512, knn 32, bf16:
    sampled tokens checked against the oracle (scores within tolerance,
    selection bit-exact from the kernel's sub-scores)."""
    N, H, n, half, knn = 16384, 8, 1024, 256, 32
    gd = torch.Generator(device=device).manual_seed(17)
    q = torch.randn((N, H, 2 * half), generator=gd, device=device).to(torch.bfloat16)
    k = ((torch.rand((2 * H * n, half), generator=gd, device=device) * 2 - 1) * half**-0.5).to(torch.bfloat16)
    scores, idx, i1, i2, s1, s2 = score_topk(q, k, H, knn, "dot", sub_outputs=True)
    torch.cuda.synchronize()
    rows = torch.randint(0, N, (96,), generator=gen(18))
    qs, kc = q[rows.to(device)].cpu(), k.cpu()
    e_s1, e_s2 = ref.sub_scores(qs, kc, H)
    assert_rel_close(s1[rows.to(device)].cpu(), e_s1, REL_TOL[torch.bfloat16], "s1")
    assert_rel_close(s2[rows.to(device)].cpu(), e_s2, REL_TOL[torch.bfloat16], "s2")
    e_scores, e_idx, _, _ = ref.select(s1[rows.to(device)].cpu(), s2[rows.to(device)].cpu(), knn)
    got_idx = idx.view(N, H, knn)[rows.to(device)].cpu()
    got_scores = scores.view(N, H, knn)[rows.to(device)].cpu()
    assert torch.equal(got_idx, e_idx) and torch.equal(got_scores, e_scores)
    # size-independent properties over every row: sorted best first, ids in
    # range and distinct per (token, head)
    sc = scores.float()
    assert bool((sc[:, :-1] >= sc[:, 1:]).all())
    assert int(idx.min()) >= 0 and int(idx.max()) < n * n
    srt = idx.sort(dim=1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("dense", [False, True], ids=["sparse", "sparse+dense"])
def test_score_grad_dense_bit_exact(device, dtype, dense):
    """pkm_score_grad_dense equals the oracle bit for bit (float32 sums in j
    order, one rounding), on selections with shared sub-keys."""
    N, H, n, half, knn = 37, 4, 512, 64, 32
    q, k = _random_inputs(N, H, n, half, dtype, seed=20)
    _, idx, _, _, _, _ = _run(q, k, H, knn, "dot", device)
    g = gen(21)
    d = torch.randn((N, H, knn), generator=g).to(dtype)
    ds1 = torch.randn((N, H, n), generator=g).to(dtype) if dense else None
    ds2 = torch.randn((N, H, n), generator=g).to(dtype) if dense else None
    got = score_grad_dense(idx.view(N * H, knn).to(device), d.view(N * H, knn).to(device), H, n,
                           ds1.to(device) if dense else None, ds2.to(device) if dense else None)
    exp = ref.score_grad_dense(idx.view(N, H, knn), d, n, ds1, ds2)
    assert torch.equal(got.cpu(), exp)


@pytest.mark.parametrize("score_type", ["dot_product", "idw"])
def test_fwpkm_drop_in(device, score_type):
    """fwpkm get_indices / compute_qk_scores drop-ins (fwpkm/fwpkm.py:853-934):
    the 6-tuple's shapes, the selection bit-exact from the returned
    sub-scores, and compute_qk_scores within tolerance of the oracle."""
    from modelos_amd.fwpkm.fwpkm import FastWeightProductKeyMemory

    m = FastWeightProductKeyMemory(mem_k_dim=256, mem_v_dim=16, mem_heads=4, mem_topk=16, mem_n_subkeys=512,
                                   qk_score_type=score_type)
    BT = 50
    q, k = _random_inputs(BT, m.heads, m.subsize, m.k_dim // 2, torch.float32, seed=22)
    scores, idx, i1, i2, s1, s2 = m.get_indices(q.to(device), k.to(device))
    assert scores.shape == idx.shape == i1.shape == i2.shape == (BT, m.heads, m.topk)
    assert s1.shape == s2.shape == (BT, m.heads, m.subsize)
    e = ref.select(s1.cpu(), s2.cpu(), m.topk)
    assert torch.equal(idx.cpu(), e[1]) and torch.equal(scores.cpu(), e[0])
    st = "dot" if score_type == "dot_product" else "idw"
    e_s1, _ = ref.sub_scores(q, k, m.heads, st)
    assert_rel_close(s1.cpu(), e_s1, REL_TOL[torch.float32], "s1")
    kv = k.view(m.heads, 2, m.subsize, m.k_dim // 2)[:, 0].contiguous().to(device)
    dense = m.compute_qk_scores(q[:, :, : m.k_dim // 2].contiguous().to(device), kv)
    # 1e-5 against each score's rounding bound: |q| . |k| for a dot product; for idw the float32
    # rounding of d^2 = |q|^2 + |k|^2 - 2 <q, k> (bounded by (|q| + |k|)^2) divided by 1e-3 + d^2
    q1 = q[:, :, : m.k_dim // 2].double()
    k1 = k.view(m.heads, 2, m.subsize, m.k_dim // 2)[:, 0].double()
    mag = torch.einsum("bhd,hnd->bhn", q1.abs(), k1.abs())
    if st == "dot":
        cond = mag
    else:
        qq, kk = (q1 * q1).sum(-1)[:, :, None], (k1 * k1).sum(-1)[None]
        d2 = (qq + kk - 2 * torch.einsum("bhd,hnd->bhn", q1, k1)).clamp_min(0.0)
        cond = (qq + kk + 2 * mag) / (1e-3 + d2) + e_s1.abs()
    assert_rel_close(dense.cpu(), e_s1, REL_TOL[torch.float32], "compute_qk_scores", cond=cond)


def test_bf16_knn_growing_in_one_process(device):
    """The cartesian step's LDS grows with knn (83 KB at knn 64): a small knn
    followed by knn 64 in the same process must both run (the kernel's LDS
    limit is raised once, to the device maximum) and match the oracle."""
    N, H, n, half = 24, 2, 1024, 128
    q, k = _int_inputs(N, H, n, half, torch.bfloat16, seed=61)
    for knn in (4, 64):
        scores, idx, _, _, _, _ = _run(q, k, H, knn, "dot", device)
        e_scores, e_idx, _, _, _, _ = ref.get_indices(q, k, H, knn)
        assert torch.equal(idx, e_idx.reshape(N * H, knn)) and torch.equal(scores, e_scores.reshape(N * H, knn)), knn
