"""GPU parity of the sparse score backward (pkm_score_grad_sparse).

d_query = dS_c @ keys_c and d_keys_c = dS_c^T @ q_c, where dS is the dense
sub-score gradient that oracle.pkm.score_grad_dense states (float32 sums in j
order, one rounding to bfloat16). Small cases are checked against float64
products of the oracle's dS; the full layer shape against float32 GEMMs of
the dense kernel's dS (which equals the oracle's bit for bit). Tolerance:
bfloat16 output, rel 2e-2 at the tensor's scale.
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd import _lib
from modelos_amd.product_keys import score_grad_dense, score_grad_sparse, score_topk
from oracle import pkm as ref
from tests.helpers import REL_TOL, assert_rel_close, gen

pytestmark = pytest.mark.gpu

TOL = REL_TOL[torch.bfloat16]

# (tokens, heads, n_keys, half, knn)
SHAPES = [
    (45, 4, 256, 64, 16),  # ragged token tile
    (300, 2, 256, 256, 64),  # knn 64, several token splits of d_keys
    (129, 3, 128, 48, 7),  # half not a multiple of 64 (partial wave tiles), odd knn
    (1, 1, 128, 16, 1),  # one token, knn 1, smallest half
    (700, 8, 1024, 256, 32),  # the PKM layer's head shape (512 x 128 dK tiles)
    (150, 2, 512, 128, 64),  # 512 x 128 dK tiles with knn 64, one dim block, ragged chunk
    (40, 1, 8448, 16, 8),  # key rows too many for the LDS slice: direct gather
]


def _ids(shape):
    return "N{}-H{}-n{}-h{}-k{}".format(*shape)


def _inputs(N, H, n, half, knn, seed):
    g = gen(seed)
    q = torch.randn((N, H, 2 * half), generator=g).to(torch.bfloat16)
    k = (torch.rand((2 * H * n, half), generator=g) * 2 - 1).mul(half**-0.5).to(torch.bfloat16)
    d = torch.randn((N * H, knn), generator=g).to(torch.bfloat16)
    return q, k, d


def _expected(q, k, idx, d, H, n):
    """float64 products of the oracle's bfloat16 dS with q and keys."""
    N, half = q.shape[0], k.shape[1]
    knn = idx.shape[-1]
    dS = ref.score_grad_dense(idx.view(N, H, knn), d.view(N, H, knn), n).double()  # [H, 2, N, n]
    Kh = k.double().view(H, 2, n, half)
    qh = q.double().view(N, H, 2, half).permute(1, 2, 0, 3)  # [H, 2, N, half]
    dq = torch.matmul(dS, Kh).permute(2, 0, 1, 3).reshape(N, H, 2 * half)
    dk = torch.matmul(dS.transpose(2, 3), qh).reshape(2 * H * n, half)
    return dq, dk


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_against_oracle(device, shape):
    N, H, n, half, knn = shape
    q, k, d = _inputs(N, H, n, half, knn, seed=40 + N)
    if half % 32 == 0:
        _, idx = score_topk(q.to(device), k.to(device), H, knn)
    else:  # outside the scoring kernel's sizes: a random cartesian selection
        g = gen(41)
        idx = (torch.randint(0, n, (N * H, knn), generator=g) * n + torch.randint(0, n, (N * H, knn), generator=g))
        idx = idx.to(device)
    dq, dk = score_grad_sparse(q.to(device), k.to(device), idx, d.to(device), H)
    torch.cuda.synchronize()
    e_dq, e_dk = _expected(q, k, idx.cpu(), d, H, n)
    assert_rel_close(dq.cpu(), e_dq, TOL, "d_query")
    assert_rel_close(dk.cpu(), e_dk, TOL, "d_keys")


def test_invalid_ids_and_shared_sub_keys(device):
    """Random ids with many shared sub-keys per row, some negative or beyond
    n_keys^2 (ignored, as in the dense kernel)."""
    N, H, n, half, knn = 200, 2, 128, 64, 32
    q, k, d = _inputs(N, H, n, half, knn, seed=50)
    g = gen(51)
    a = torch.randint(0, 6, (N * H, knn), generator=g)
    b = torch.randint(0, n, (N * H, knn), generator=g)
    idx = a * n + b
    bad = torch.rand((N * H, knn), generator=g) < 0.1
    idx = torch.where(bad, torch.where(torch.rand((N * H, knn), generator=g) < 0.5, -1, n * n + 5), idx)
    dq, dk = score_grad_sparse(q.to(device), k.to(device), idx.to(device), d.to(device), H)
    torch.cuda.synchronize()
    # expected: the valid ids only (an invalid one becomes id 0 with gradient 0)
    e_dq, e_dk = _expected(q, k, torch.where(bad, 0, idx), torch.where(bad, 0.0, d.float()).to(d.dtype), H, n)
    assert_rel_close(dq.cpu(), e_dq, TOL, "d_query")
    assert_rel_close(dk.cpu(), e_dk, TOL, "d_keys")


def test_one_gradient_only_and_deterministic(device):
    N, H, n, half, knn = 257, 4, 256, 128, 32
    q, k, d = _inputs(N, H, n, half, knn, seed=60)
    qd, kd, dd = q.to(device), k.to(device), d.to(device)
    _, idx = score_topk(qd, kd, H, knn)
    dq, dk = score_grad_sparse(qd, kd, idx, dd, H)
    dq_only, none_k = score_grad_sparse(qd, kd, idx, dd, H, need_keys=False)
    none_q, dk_only = score_grad_sparse(qd, kd, idx, dd, H, need_query=False)
    dq2, dk2 = score_grad_sparse(qd, kd, idx, dd, H)
    torch.cuda.synchronize()
    assert none_k is None and none_q is None
    assert torch.equal(dq_only, dq) and torch.equal(dk_only, dk)
    assert torch.equal(dq2, dq) and torch.equal(dk2, dk)


def test_empty_tokens(device):
    H, n, half, knn = 2, 128, 64, 8
    q = torch.zeros((0, H, 2 * half), dtype=torch.bfloat16, device=device)
    k = torch.randn((2 * H * n, half), device=device).to(torch.bfloat16)
    idx = torch.zeros((0, knn), dtype=torch.long, device=device)
    d = torch.zeros((0, knn), dtype=torch.bfloat16, device=device)
    dq, dk = score_grad_sparse(q, k, idx, d, H)
    torch.cuda.synchronize()
    assert dq.shape == (0, H, 2 * half)
    assert not bool(dk.any())


@pytest.mark.parametrize(
    "n,half,knn",
    [(192, 64, 8), (128, 272, 8), (128, 40, 8), (128, 64, 65)],
    ids=["n-not-128", "half-too-big", "half-not-16", "knn-65"],
)
def test_unsupported_sizes(device, n, half, knn):
    """Sizes outside the kernel's limits: the wrapper returns None (the
    autograd backward then takes the dense path) and the C entry point
    refuses them."""
    H = 1
    q = torch.randn((4, H, 2 * half), device=device).to(torch.bfloat16)
    k = torch.randn((2 * H * n, half), device=device).to(torch.bfloat16)
    idx = torch.zeros((4 * H, knn), dtype=torch.long, device=device)
    d = torch.zeros((4 * H, knn), dtype=torch.bfloat16, device=device)
    assert score_grad_sparse(q, k, idx, d, H) is None
    with pytest.raises(_lib.PkmError):
        _lib.call("pkm_score_grad_sparse", _lib.ptr(idx), _lib.ptr(d), _lib.dtype_code(d), 4, H, n, half, knn,
                  _lib.ptr(q), _lib.ptr(k), _lib.ptr(q), _lib.ptr(k), None, 0, _lib.stream_of(q.device))


def test_full_layer_shape(device):
    """16384 tokens x 8 heads, 1024 keys per half, half 256, knn 32: against
    float32 GEMMs of the dense sub-score gradient (bit-exact with the oracle's)."""
    N, H, n, half, knn = 16384, 8, 1024, 256, 32
    gd = torch.Generator(device=device).manual_seed(70)
    q = torch.randn((N, H, 2 * half), generator=gd, device=device).to(torch.bfloat16)
    k = ((torch.rand((2 * H * n, half), generator=gd, device=device) * 2 - 1) * half**-0.5).to(torch.bfloat16)
    d = torch.randn((N * H, knn), generator=gd, device=device).to(torch.bfloat16)
    _, idx = score_topk(q, k, H, knn)
    dq, dk = score_grad_sparse(q, k, idx, d, H)
    dS = score_grad_dense(idx, d, H, n).float().view(2 * H, N, n)
    Kh = k.float().view(2 * H, n, half)
    qh = q.float().view(N, H, 2, half).permute(1, 2, 0, 3).reshape(2 * H, N, half).contiguous()
    e_dq = torch.bmm(dS, Kh).view(H, 2, N, half).permute(2, 0, 1, 3).reshape(N, H, 2 * half)
    e_dk = torch.bmm(dS.transpose(1, 2).contiguous(), qh).reshape(2 * H * n, half)
    torch.cuda.synchronize()
    assert_rel_close(dq, e_dq, TOL, "d_query")
    assert_rel_close(dk, e_dk, TOL, "d_keys")
