"""Pins the embedding-bag oracle (oracle/eb.py) against independent checks:
F.embedding_bag and its autograd (library routines), fp64 gradcheck /
gradgradcheck (numerical differentiation), brute-force loops and closed forms.
CPU only."""
import pytest
import torch
import torch.nn.functional as F

from oracle import eb as ref
from tests.helpers import assert_rel_close, eb_inputs, gen


@pytest.mark.parametrize("B,L,K,D", [(5, 3, 7, 4), (16, 32, 50, 16), (3, 1, 2, 8)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_forward_matches_library_embedding_bag(B, L, K, D, dtype):
    W, idx, p, _ = eb_inputs(B, L, K, D, dtype, seed=1, softmax=False, with_grad=False)
    got = ref.eb_forward(idx, W, p)
    lib = F.embedding_bag(idx, W, per_sample_weights=p, mode="sum")
    assert_rel_close(got, lib, 1e-12 if dtype == torch.float64 else 1e-6, "forward vs F.embedding_bag")


def test_forward_matches_brute_force():
    W, idx, p, _ = eb_inputs(4, 6, 9, 5, torch.float64, seed=2, softmax=False, with_grad=False)
    assert_rel_close(ref.eb_forward(idx, W, p), ref.brute_force_forward(idx, W, p), 1e-12, "forward vs loops")
    assert_rel_close(ref.eb_forward(idx, W, None), ref.brute_force_forward(idx, W, None), 1e-12, "unweighted")


def test_forward_closed_forms():
    W, idx, _, _ = eb_inputs(8, 1, 13, 6, torch.float64, seed=3, psw=False, with_grad=False)
    # a single-entry bag with weight 1 copies the row
    assert torch.equal(ref.eb_forward(idx, W, torch.ones(8, 1, dtype=torch.float64)), W[idx[:, 0]])
    # a bag of one row repeated k times with weights w sums to (sum w) * row
    r = torch.full((3, 5), 4, dtype=torch.long)
    w = torch.rand((3, 5), generator=gen(4), dtype=torch.float64)
    assert_rel_close(ref.eb_forward(r, W, w), w.sum(1, keepdim=True) * W[4], 1e-14, "repeated row")
    # linearity in the weights
    W2, idx2, p1, _ = eb_inputs(6, 4, 10, 3, torch.float64, seed=5, softmax=False, with_grad=False)
    p2 = torch.randn(p1.shape, generator=gen(6), dtype=torch.float64)
    lhs = ref.eb_forward(idx2, W2, 2.0 * p1 - 3.0 * p2)
    rhs = 2.0 * ref.eb_forward(idx2, W2, p1) - 3.0 * ref.eb_forward(idx2, W2, p2)
    assert_rel_close(lhs, rhs, 1e-12, "linearity")


def test_forward_bf16_rounds_once_from_float32():
    W, idx, p, _ = eb_inputs(7, 9, 11, 16, torch.bfloat16, seed=7, with_grad=False)
    exact = ref.eb_forward(idx, W.double(), p.double())
    got = ref.eb_forward(idx, W, p)
    assert got.dtype == torch.bfloat16
    # one rounding of a float32 sum: within a bf16 half-ulp plus float32 error
    assert ((got.double() - exact).abs() <= exact.abs() * 2**-8 + 1e-6).all()


def test_forward_invalid_indices_contribute_nothing():
    W, idx, p, _ = eb_inputs(4, 5, 6, 3, torch.float64, seed=8, softmax=False, with_grad=False)
    bad = idx.clone()
    bad[0, 1] = -1
    bad[2, 4] = 6
    keep = torch.ones_like(p)
    keep[0, 1] = 0
    keep[2, 4] = 0
    assert_rel_close(ref.eb_forward(bad, W, p), ref.eb_forward(idx, W, p * keep), 1e-14, "invalid rows")


@pytest.mark.parametrize("with_psw", [True, False])
def test_backward_matches_autograd_of_library(with_psw):
    W, idx, p, g = eb_inputs(6, 5, 8, 4, torch.float64, seed=9, psw=with_psw, softmax=False)
    Wr = W.clone().requires_grad_(True)
    pr = p.clone().requires_grad_(True) if with_psw else None
    out = F.embedding_bag(idx, Wr, per_sample_weights=pr, mode="sum")
    grads = torch.autograd.grad(out, [Wr] + ([pr] if with_psw else []), g)
    gW, gp = ref.eb_backward(idx, W, p, g)
    assert_rel_close(gW, grads[0], 1e-12, "gW vs autograd")
    if with_psw:
        assert_rel_close(gp, grads[1], 1e-12, "gpsw vs autograd")
    else:
        assert gp is None


def test_backward_matches_brute_force_and_gradcheck():
    W, idx, p, g = eb_inputs(4, 7, 5, 3, torch.float64, seed=10, softmax=False)
    gW, gp = ref.eb_backward(idx, W, p, g)
    bW, bp = ref.brute_force_backward(idx, W, p, g)
    assert_rel_close(gW, bW, 1e-12, "gW vs loops")
    assert_rel_close(gp, bp, 1e-12, "gpsw vs loops")
    # the oracle forward's own derivative is the numerical derivative
    Wr = W.clone().requires_grad_(True)
    pr = p.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda w_, p_: ref.eb_forward(idx, w_, p_), (Wr, pr))
    # and equals the oracle backward
    out = ref.eb_forward(idx, Wr, pr)
    aW, ap = torch.autograd.grad(out, (Wr, pr), g)
    assert_rel_close(gW, aW, 1e-12, "gW vs autograd of oracle forward")
    assert_rel_close(gp, ap, 1e-12, "gpsw vs autograd of oracle forward")


def test_backward_untouched_rows_are_zero_and_column_sums():
    W, idx, p, g = eb_inputs(10, 3, 40, 4, torch.float64, seed=11, softmax=False)
    gW, _ = ref.eb_backward(idx, W, p, g)
    untouched = torch.ones(40, dtype=torch.bool)
    untouched[idx.reshape(-1)] = False
    assert untouched.any() and (gW[untouched] == 0).all()
    # checksum: sum over rows of gW = sum_b (sum_j w[b,j]) g[b]
    assert_rel_close(gW.sum(0), (p.sum(1, keepdim=True) * g).sum(0), 1e-12, "column sums")


def _diff_weight_grad(idx, a, g, K):
    """Differentiable restatement of the first-order weight gradient (index_add_)."""
    B, L = idx.shape
    D = g.shape[1]
    contrib = (g[:, None, :] * (a[:, :, None] if a is not None else 1.0)).expand(B, L, D).reshape(B * L, D)
    return torch.zeros(K, D, dtype=g.dtype).index_add(0, idx.reshape(-1), contrib)


@pytest.mark.parametrize("with_a", [True, False])
def test_double_backward_matches_autograd(with_a):
    K = 9
    W, idx, a, g = eb_inputs(5, 4, K, 3, torch.float64, seed=12, psw=with_a, softmax=False)
    gbar = torch.randn((K, 3), generator=gen(13), dtype=torch.float64)
    gr = g.clone().requires_grad_(True)
    ar = a.clone().requires_grad_(True) if with_a else None
    gw = _diff_weight_grad(idx, ar, gr, K)
    inputs = [gr] + ([ar] if with_a else [])
    want = torch.autograd.grad(gw, inputs, gbar)
    d_g, d_a = ref.eb_double_backward(idx, a, g, gbar)
    assert_rel_close(d_g, want[0], 1e-12, "d_grad_output")
    if with_a:
        assert_rel_close(d_a, want[1], 1e-12, "d_a")
    bg, ba = ref.brute_force_double_backward(idx, a, g, gbar)
    assert_rel_close(d_g, bg, 1e-12, "d_grad_output vs loops")
    if with_a:
        assert_rel_close(d_a, ba, 1e-12, "d_a vs loops")


def test_double_backward_gradgradcheck():
    K = 6
    W, idx, a, g = eb_inputs(3, 4, K, 2, torch.float64, seed=14, softmax=False)
    Wr = W.clone().requires_grad_(True)
    ar = a.clone().requires_grad_(True)
    assert torch.autograd.gradgradcheck(lambda w_, a_: ref.eb_forward(idx, w_, a_), (Wr, ar))
