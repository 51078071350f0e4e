"""Parity of the HIP embedding-bag kernels (through the C ABI) with the oracle.

Small and ragged sizes are compared element-wise with oracle/eb.py on the same
seeded inputs; the full standalone size (16384 bags x 128 lookups into a
2^20 x 1024 bf16 table) is checked on sampled bags / rows against the oracle
plus size-independent properties (column-sum checksum, untouched rows exactly
zero, bitwise run-to-run determinism). Tolerances: 1e-5 relative (fp32),
2e-2 (bf16), 2e-3 (fp16), relative to each tensor's scale.
"""
import pytest
import torch

from oracle import eb as ref
from tests.helpers import REL_TOL, assert_rel_close, eb_inputs

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]

# (B, L, K, D): row lengths hit every lane-group shape (LPG 1..64, VPL 1..8),
# bag sizes around the 64-entry batch, tiny and empty cases.
SHAPES = [
    (33, 17, 1000, 1024),
    (7, 64, 500, 512),
    (9, 65, 300, 256),
    (5, 128, 2000, 2048),
    (3, 3, 50, 4096),
    (17, 31, 100, 128),
    (21, 5, 64, 64),
    (4, 2, 10, 32),
    (6, 1, 9, 16),
    (2, 7, 40, 8),
]


def _dev(*ts, device):
    return [t.to(device) if t is not None else None for t in ts]


def _reduce_supported(D, dtype):
    """The backward / double-backward kernels hold a whole row per lane group:
    dim / (16 B / element size) must be LPG * VPL with VPL <= 8."""
    epv = 4 if dtype == torch.float32 else 8
    return (D // epv) <= 512


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("B,L,K,D", SHAPES)
def test_forward_parity(B, L, K, D, dtype, device):
    from modelos_amd import embedding_bag as eb

    if dtype == torch.float32 and D == 8:
        D = 12  # not a multiple of 8 for 16-bit, exercises fp32 LPG=1; 16-bit uses the scalar fallback below
    W, idx, p, _ = eb_inputs(B, L, K, D, dtype, seed=B * 1000 + L, with_grad=False)
    out = eb.eb_forward(*_dev(idx, W, p, device=device))
    assert out.dtype == dtype and out.shape == (B, D)
    assert_rel_close(out, ref.eb_forward(idx, W, p), REL_TOL[dtype], f"forward {dtype} {B,L,K,D}")


@pytest.mark.parametrize("D", [12, 20, 6])
def test_forward_scalar_fallback(D, device):
    from modelos_amd import embedding_bag as eb

    W, idx, p, _ = eb_inputs(5, 9, 30, D, torch.bfloat16, seed=D, with_grad=False)
    out = eb.eb_forward(*_dev(idx, W, p, device=device))
    assert_rel_close(out, ref.eb_forward(idx, W, p), 2e-2, "scalar fallback")


def test_forward_unweighted_mixed_dtypes_and_invalid(device):
    from modelos_amd import embedding_bag as eb

    W, idx, p, _ = eb_inputs(19, 40, 700, 1024, torch.bfloat16, seed=5, psw_dtype=torch.float32, with_grad=False)
    idx[0, 0] = -5
    idx[3, 39] = 700
    idx[7, 12] = 1 << 40
    dW, didx, dp = _dev(W, idx, p, device=device)
    assert_rel_close(eb.eb_forward(didx, dW, dp), ref.eb_forward(idx, W, p), 2e-2, "fp32 psw on bf16 table")
    assert_rel_close(eb.eb_forward(didx, dW, None), ref.eb_forward(idx, W, None), 2e-2, "unweighted")
    assert eb.count_invalid_indices(didx, 700) == 3


def test_forward_empty(device):
    from modelos_amd import embedding_bag as eb

    W = torch.randn(10, 64, device=device)
    assert eb.eb_forward(torch.zeros(0, 3, dtype=torch.long, device=device), W, None).shape == (0, 64)
    out = eb.eb_forward(torch.zeros(4, 0, dtype=torch.long, device=device), W, torch.zeros(4, 0, device=device))
    assert (out == 0).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("B,L,K,D", SHAPES)
def test_backward_parity(B, L, K, D, dtype, device):
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = eb_inputs(B, L, K, D, dtype, seed=B * 7 + L)
    if not _reduce_supported(D, dtype):
        from modelos_amd._lib import PkmError

        with pytest.raises(PkmError, match="not supported"):
            eb.eb_backward(*_dev(idx, W, p, g, device=device))
        return
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    eW, ep = ref.eb_backward(idx, W, p, g)
    assert gW.dtype == dtype and gp.dtype == p.dtype
    assert_rel_close(gW, eW, REL_TOL[dtype], f"grad_weight {dtype} {B,L,K,D}")
    assert_rel_close(gp, ep, REL_TOL[dtype], f"grad_psw {dtype} {B,L,K,D}")


def _hot_indices(B, L, K, seed):
    """Indices with heavy rows: row 3 takes ~1/3 of all lookups, rows 4 and 5
    ~600 each (adjacent heavy rows share chunks), the rest uniform, plus a few
    out-of-range entries."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, K, (B, L), generator=g)
    u = torch.rand((B, L), generator=g)
    idx[u < 1 / 3] = 3
    flat = idx.view(-1)
    pos = torch.randperm(B * L, generator=g)
    flat[pos[:600]] = 4
    flat[pos[600:1200]] = 5
    flat[pos[1200:1205]] = -1
    return idx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("D", [1024, 64])
def test_backward_heavy_rows(D, dtype, device):
    from modelos_amd import embedding_bag as eb

    B, L, K = 97, 64, 5000
    W, _, p, g = eb_inputs(B, L, K, D, dtype, seed=21)
    idx = _hot_indices(B, L, K, seed=22)
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    eW, ep = ref.eb_backward(idx, W, p, g)
    assert_rel_close(gW, eW, REL_TOL[dtype], "heavy grad_weight")
    assert_rel_close(gp, ep, REL_TOL[dtype], "heavy grad_psw")
    assert (gp.cpu()[idx < 0] == 0).all()


def test_backward_unweighted_and_deterministic(device):
    from modelos_amd import embedding_bag as eb

    W, idx, _, g = eb_inputs(64, 48, 3000, 512, torch.float32, seed=23, psw=False)
    idx = _hot_indices(64, 48, 3000, seed=24)
    dW, didx, dg = _dev(W, idx, g, device=device)
    gW1, gp1 = eb.eb_backward(didx, dW, None, dg)
    gW2, _ = eb.eb_backward(didx, dW, None, dg)
    assert gp1 is None
    eW, _ = ref.eb_backward(idx, W, None, g)
    assert_rel_close(gW1, eW, 1e-5, "unweighted grad_weight")
    assert torch.equal(gW1, gW2), "backward is not bitwise deterministic"


def test_backward_empty_bags_zero_grad(device):
    from modelos_amd import embedding_bag as eb

    W = torch.randn(100, 256, device=device)
    gW, gp = eb.eb_backward(
        torch.zeros(0, 4, dtype=torch.long, device=device), W, torch.zeros(0, 4, device=device),
        torch.zeros(0, 256, device=device),
    )
    assert (gW == 0).all() and gp.shape == (0, 4)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("B,L,K,D", SHAPES)
@pytest.mark.parametrize("with_a", [True, False])
def test_double_backward_parity(B, L, K, D, dtype, with_a, device):
    from modelos_amd import embedding_bag as eb

    _, idx, a, g = eb_inputs(B, L, K, D, dtype, seed=B + L + D, psw=with_a)
    gbar = torch.randn((K, D), generator=torch.Generator().manual_seed(3)).to(dtype)
    if not _reduce_supported(D, dtype):
        from modelos_amd._lib import PkmError

        with pytest.raises(PkmError, match="not supported"):
            eb.eb_double_backward(*_dev(idx, a, g, gbar, device=device))
        return
    d_g, d_a = eb.eb_double_backward(*_dev(idx, a, g, gbar, device=device))
    e_g, e_a = ref.eb_double_backward(idx, a, g, gbar)
    assert_rel_close(d_g, e_g, REL_TOL[dtype], f"d_grad_output {dtype}")
    if with_a:
        assert_rel_close(d_a, e_a, REL_TOL[dtype], f"d_a {dtype}")
    else:
        assert d_a is None


def _bits_equal_fraction(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.cpu() == b.cpu()).float().mean().item()


@pytest.mark.parametrize("D", [512, 1024, 64, 4096])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_backward_float32_gradient_into_half_table(dtype, D, device):
    """A float32 upstream gradient into a 16-bit table is read as float32,
    as the reference's kernel reads it (pkm/xformer_embeddingbag.py:322):
    the table gradient is the float32 sum of the unrounded products, rounded
    once, so it equals the float64 sum rounded to the table dtype except where
    that sum lies within float32 rounding of a rounding boundary (rounding the
    gradient to the table dtype first moves about a third of the entries)."""
    from modelos_amd import embedding_bag as eb

    B, L, K = 48, 32, 700
    W, idx, p, _ = eb_inputs(B, L, K, D, dtype, seed=77, psw_dtype=torch.float32, with_grad=False)
    g = torch.randn((B, D), generator=torch.Generator().manual_seed(78))
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    e64W, e64p = ref.eb_backward(idx, W.double(), p.double(), g.double())
    assert gW.dtype == dtype and gp.dtype == torch.float32
    assert _bits_equal_fraction(gW, e64W.to(dtype)) > 0.999
    cW = ref.eb_backward(idx, W.double().abs(), p.double().abs(), g.double().abs())[0]
    # one rounding to the table dtype (half a unit in the last place; float16's subnormals have a
    # fixed spacing of 2^-24)
    assert_rel_close(gW, e64W, 2 ** -8 if dtype == torch.bfloat16 else 2 ** -11, "grad_weight", cond=cW,
                     atol=2 ** -25 if dtype == torch.float16 else 0.0)
    # psw-gradient: a float32 dot of the table row (exact in float32) and the float32 gradient
    cp = ref.eb_backward(idx, W.double().abs(), p.double().abs(), g.double().abs())[1]
    assert_rel_close(gp, e64p, 1e-5, "grad_psw", cond=cp)
    # the same through the fixed-scratch entry point
    from modelos_amd import _lib

    dW, didx, dp, dg = _dev(W, idx, p, g, device=device)
    gW2 = torch.empty_like(dW)
    gp2 = torch.empty_like(dp)
    _lib.call("pkm_eb_bwd_noalloc", _lib.ptr(dW), K, D, _lib.dtype_code(dW), _lib.ptr(didx), _lib.ptr(dp),
              _lib.dtype_code(dp), _lib.ptr(dg), _lib.dtype_code(dg), B, L, _lib.ptr(gW2), _lib.ptr(gp2),
              _lib.stream_of(dW.device))
    torch.cuda.synchronize()
    assert torch.equal(gW2, gW) and torch.equal(gp2, gp)


@pytest.mark.parametrize("gdt", [torch.float16, torch.bfloat16], ids=str)
def test_backward_gradient_of_other_dtype(gdt, device):
    """A 16-bit gradient into a float32 table, or a 16-bit gradient of the
    other 16-bit type: read as float32 (exact widening), so the result is the
    reference's float32 computation on those gradient values."""
    from modelos_amd import embedding_bag as eb

    B, L, K, D = 40, 16, 500, 256
    for wdt in (torch.float32, torch.bfloat16 if gdt == torch.float16 else torch.float16):
        W, idx, p, _ = eb_inputs(B, L, K, D, wdt, seed=81, psw_dtype=torch.float32, with_grad=False)
        g = torch.randn((B, D), generator=torch.Generator().manual_seed(82)).to(gdt)
        gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
        e64W, e64p = ref.eb_backward(idx, W.double(), p.double(), g.double())
        assert gW.dtype == wdt
        cW = ref.eb_backward(idx, W.double().abs(), p.double().abs(), g.double().abs())[0]
        if wdt == torch.float32:
            assert_rel_close(gW, e64W, 1e-6, f"grad_weight {wdt} <- {gdt}", cond=cW)
        else:
            assert _bits_equal_fraction(gW, e64W.to(wdt)) > 0.999
        assert_rel_close(gp, e64p, 1e-5, f"grad_psw {wdt} <- {gdt}",
                         cond=ref.eb_backward(idx, W.double().abs(), p.double().abs(), g.double().abs())[1])


@pytest.mark.parametrize("gbar_dt,g_dt", [(torch.bfloat16, torch.float32), (torch.float16, torch.float32),
                                          (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float16)],
                         ids=lambda v: str(v).replace("torch.", ""))
def test_double_backward_table_gradient_dtype_differs(gbar_dt, g_dt, device):
    """g_bar (the gradient of the table gradient) and the upstream gradient
    in different dtypes: g_bar [K, D] is read in its own dtype (no copy), the
    upstream gradient in its own dtype or as float32, the sums in float32
    (the reference's type promotion), d_grad_output returned in the upstream
    gradient's dtype (as autograd returns it)."""
    from modelos_amd import embedding_bag as eb

    B, L, K, D = 40, 24, 600, 256
    _, idx, a, g = eb_inputs(B, L, K, D, torch.float32, seed=79)
    g = g.to(g_dt)
    gbar = torch.randn((K, D), generator=torch.Generator().manual_seed(80)).to(gbar_dt)
    d_g, d_a = eb.eb_double_backward(*_dev(idx, a, g, gbar, device=device))
    e_g, e_a = ref.eb_double_backward(idx, a.double(), g.double(), gbar.double())
    c_g, c_a = ref.eb_double_backward(idx, a.double().abs(), g.double().abs(), gbar.double().abs())
    assert d_g.dtype == g_dt and d_a.dtype == a.dtype
    tol_g = 1e-5 if g_dt == torch.float32 else REL_TOL[g_dt]
    assert_rel_close(d_g, e_g, tol_g, "d_grad_output", cond=c_g)
    assert_rel_close(d_a, e_a, 1e-5, "d_a", cond=c_a)
    if g_dt != torch.float32:
        # the float32 sums round once: equal to the float64 result rounded to the output dtype
        assert _bits_equal_fraction(d_g, e_g.to(g_dt)) > 0.99


def test_autograd_dropin_pkm(device):
    from modelos_amd.pkm.xformer_embeddingbag import xformers_embedding_bag

    W, idx, p, g = eb_inputs(40, 32, 900, 1024, torch.bfloat16, seed=31)
    dW, didx, dp, dg = _dev(W, idx, p, g, device=device)
    dW.requires_grad_(True)
    dp.requires_grad_(True)
    out = xformers_embedding_bag(didx, dW, dp)
    out.backward(dg)
    eW, ep = ref.eb_backward(idx, W, p, g)
    assert_rel_close(out, ref.eb_forward(idx, W, p), 2e-2, "pkm drop-in forward")
    assert_rel_close(dW.grad, eW, 2e-2, "pkm drop-in weight grad")
    assert_rel_close(dp.grad, ep, 2e-2, "pkm drop-in psw grad")


@pytest.mark.parametrize("bw_algo", ["atomics", "lock"])
def test_dispatcher_bw_algo_variants(bw_algo, device):
    """xformers_embedding_bag(..., bw_algo=...) (pkm/xformer_embeddingbag.py:403-438):
    the atomics and lock variants give the reverse-indices gradients bit for
    bit (all three run the deterministic backward; the reference's "lock"
    variant returns an all-zero table gradient, a bug not reproduced), and
    match the oracle."""
    from modelos_amd.pkm.xformer_embeddingbag import xformers_embedding_bag

    W, idx, p, g = eb_inputs(64, 48, 2000, 512, torch.bfloat16, seed=37)
    idx[:, :6] = 11  # a hot row
    grads = {}
    for algo in ("reverse_indices", bw_algo):
        dW, didx, dp, dg = _dev(W, idx, p, g, device=device)
        dW.requires_grad_(True)
        dp.requires_grad_(True)
        xformers_embedding_bag(didx, dW, dp, bw_algo=algo).backward(dg)
        grads[algo] = (dW.grad.cpu(), dp.grad.cpu())
    assert torch.equal(grads[bw_algo][0], grads["reverse_indices"][0])
    assert torch.equal(grads[bw_algo][1], grads["reverse_indices"][1])
    eW, ep = ref.eb_backward(idx, W, p, g)
    assert_rel_close(grads[bw_algo][0], eW, 2e-2, f"{bw_algo} weight grad", cond=ref.eb_backward(idx, W.abs(), p.abs(), g.abs())[0])
    assert_rel_close(grads[bw_algo][1], ep, 2e-2, f"{bw_algo} psw grad")


def test_autograd_dropin_fwpkm_double_backward(device):
    """Outer gradient through one inner SGD step on the table, the fwpkm pattern
    (fwpkm/fwpkm.py:308-365): compared with the same computation done by
    autograd on the oracle's differentiable forward in float64."""
    from modelos_amd.fwpkm.xformer_embeddingbag_grad_wrapper import xformers_embedding_bag

    B, L, K, D = 24, 16, 300, 256
    W, idx, a, _ = eb_inputs(B, L, K, D, torch.float32, seed=41)
    tgt = torch.randn((B, D), generator=torch.Generator().manual_seed(42))
    idx2 = torch.randint(0, K, (B, L), generator=torch.Generator().manual_seed(43))
    a2 = torch.softmax(torch.randn((B, L), generator=torch.Generator().manual_seed(44)), -1)

    def run(eb_fn, W0, a0, dev_or_none):
        hyp = eb_fn(idx if dev_or_none is None else idx.to(dev_or_none), W0, a0)
        t = tgt if dev_or_none is None else tgt.to(dev_or_none)
        inner = 0.5 * ((hyp - t) ** 2).mean()
        (gV,) = torch.autograd.grad(inner, W0, create_graph=True)
        W1 = W0 - 0.1 * gV * (B * D)
        i2 = idx2 if dev_or_none is None else idx2.to(dev_or_none)
        p2 = a2 if dev_or_none is None else a2.to(dev_or_none)
        out = eb_fn(i2, W1, p2)
        return (out**2).sum()

    Wd = W.to(device).requires_grad_(True)
    ad = a.to(device).requires_grad_(True)
    loss = run(lambda i, w, p: xformers_embedding_bag(i, w, p), Wd, ad, device)
    gW, ga = torch.autograd.grad(loss, (Wd, ad))

    We = W.double().requires_grad_(True)
    ae = a.double().requires_grad_(True)
    loss_e = run(lambda i, w, p: ref.eb_forward(i, w, p.double()), We, ae, None)
    eW, ea = torch.autograd.grad(loss_e, (We, ae))
    assert_rel_close(loss.detach(), loss_e.detach(), 1e-5, "outer loss")
    assert_rel_close(gW, eW, 1e-5, "outer grad wrt table")
    assert_rel_close(ga, ea, 1e-5, "outer grad wrt per-sample weights")


# ---------------------------------------------------------------------------
# Full standalone size: 16384 bags x 128 lookups, 2^20 x 1024 bf16 table
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def full_case(device):
    B, L, K, D = 16384, 128, 1 << 20, 1024
    g = torch.Generator(device=device).manual_seed(0)
    W = (torch.randn((K, D), generator=g, device=device) * 0.03).to(torch.bfloat16)
    idx = torch.randint(0, K, (B, L), generator=g, device=device)
    p = torch.softmax(torch.randn((B, L), generator=g, device=device), -1).to(torch.bfloat16)
    gr = torch.randn((B, D), generator=g, device=device).to(torch.bfloat16)
    return W, idx, p, gr


def test_full_size_forward_sampled(full_case):
    from modelos_amd import embedding_bag as eb

    W, idx, p, _ = full_case
    out = eb.eb_forward(idx, W, p)
    sel = torch.randperm(idx.shape[0], generator=torch.Generator().manual_seed(1))[:256].to(idx.device)
    si, sp = idx[sel].cpu(), p[sel].cpu()
    rows = W[si.reshape(-1)].cpu()
    local = torch.arange(si.numel()).view(si.shape)
    expect = ref.eb_forward(local, rows, sp)
    assert_rel_close(out[sel], expect, 2e-2, "full-size forward (sampled bags)")


def test_full_size_backward_sampled_and_properties(full_case):
    from modelos_amd import embedding_bag as eb

    W, idx, p, gr = full_case
    K, D = W.shape
    gW, gp = eb.eb_backward(idx, W, p, gr)
    gW2, gp2 = eb.eb_backward(idx, W, p, gr)
    assert torch.equal(gW, gW2) and torch.equal(gp, gp2), "not bitwise deterministic"
    # untouched rows exactly zero
    touched = torch.zeros(K, dtype=torch.bool, device=idx.device)
    touched[idx.reshape(-1)] = True
    assert (gW[~touched] == 0).all()
    # checksum over all rows: sum_r gW[r] = sum_b (sum_j p[b,j]) g[b]
    colsum = gW.float().sum(0)
    expect = (p.float().sum(1, keepdim=True) * gr.float()).sum(0)
    assert_rel_close(colsum, expect, 2e-2, "column-sum checksum")
    # sampled rows against the oracle
    rows = torch.randperm(K, generator=torch.Generator().manual_seed(2))[:512].to(idx.device)
    flat = idx.reshape(-1)
    hit = torch.isin(flat, rows)
    pos = hit.nonzero().squeeze(1)
    b = pos // idx.shape[1]
    occ_rows = flat[pos]
    contrib = p.reshape(-1)[pos].float()[:, None] * gr[b].float()
    exp_rows = torch.zeros(K, D, device=idx.device).index_add_(0, occ_rows, contrib)[rows]
    assert_rel_close(gW[rows], exp_rows, 2e-2, "sampled grad_weight rows")
    # sampled psw gradients
    sb = torch.randperm(idx.shape[0], generator=torch.Generator().manual_seed(3))[:128].to(idx.device)
    e_gp = (W[idx[sb]].float() * gr[sb].float()[:, None, :]).sum(-1)
    assert_rel_close(gp[sb], e_gp, 2e-2, "sampled grad_psw")


# Upstream gradients larger than the L2 of one XCD (the g rows of every
# occurrence are re-read from the Infinity Cache): full parity at moderate
# sizes, with heavy rows, invalid indices, unweighted bags and bitwise
# determinism.
LARGE_G = [
    (4200, 16, 50000, 1024, torch.bfloat16),  # 8.6 MB of upstream gradient
    (2200, 24, 20000, 2048, torch.bfloat16),
    (2200, 8, 30000, 1024, torch.float32),
    (8800, 4, 9000, 512, torch.float16),
]


@pytest.mark.parametrize("B,L,K,D,dtype", LARGE_G, ids=lambda v: str(v).replace("torch.", ""))
def test_backward_large_gradient_parity(B, L, K, D, dtype, device):
    from modelos_amd import embedding_bag as eb

    assert B * D * torch.tensor([], dtype=dtype).element_size() > 8 << 20
    W, _, p, g = eb_inputs(B, L, K, D, dtype, seed=31 + D)
    idx = _hot_indices(B, L, K, seed=32 + D)
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    eW, ep = ref.eb_backward(idx, W, p, g)
    # hot rows sum thousands of terms: elementwise against the sums of |terms|
    cW, cp = ref.eb_backward(idx, W.abs(), p.abs(), g.abs())
    assert_rel_close(gW, eW, REL_TOL[dtype], "grad_weight", cond=cW)
    assert_rel_close(gp, ep, REL_TOL[dtype], "grad_psw", cond=cp)
    assert (gp.cpu()[idx < 0] == 0).all()
    gW2, gp2 = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    assert torch.equal(gW, gW2) and torch.equal(gp, gp2)


# Hot rows of a bf16 table with 64-lane rows (at least max(257, bags / 16)
# lookups) are reduced as dense products on the matrix cores, their weights
# merged per bag. Rows in ~40% of the bags, a row held up to three times by one
# bag, a row at exactly the threshold and one just below it, a hot last row,
# a bag count that is not a multiple of the 32-bag chunk or the 128-bag tile,
# bf16 and float32 weights: elementwise against the oracle's sums of |terms|,
# and bitwise run-to-run.
def _hot_matrix_indices(B, L, K, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(20, K - 1, (B, L), generator=g)
    idx[torch.rand(B, generator=g) < 0.4, 0] = 7
    v = torch.rand(B, generator=g)
    idx[v < 0.3, 1] = 8
    idx[v < 0.1, 2] = 8
    idx[v < 0.05, 3] = 8
    hot_min = max(257, B // 16)
    bags = torch.randperm(B, generator=g)
    idx[bags[:hot_min], 4] = 9
    idx[bags[:hot_min - 1], 5] = 10
    idx[torch.rand(B, generator=g) < 0.5, 6] = K - 1
    idx[bags[-3:], 7] = -1
    return idx


@pytest.mark.parametrize("psw_dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("B,L,K,D", [(2000, 12, 30000, 512), (1000, 16, 5000, 2048), (4100, 8, 9000, 1024),
                                     (1000, 8, 3000, 4096)])
def test_backward_hot_rows_matrix_cores(B, L, K, D, psw_dtype, device):
    from modelos_amd import embedding_bag as eb

    W, _, p, g = eb_inputs(B, L, K, D, torch.bfloat16, seed=41 + D, psw_dtype=psw_dtype)
    idx = _hot_matrix_indices(B, L, K, seed=42 + D)
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    eW, ep = ref.eb_backward(idx, W, p, g)
    cW, cp = ref.eb_backward(idx, W.abs(), p.abs(), g.abs())
    assert_rel_close(gW, eW, REL_TOL[torch.bfloat16], "grad_weight", cond=cW)
    assert_rel_close(gp, ep, 1e-4 if psw_dtype == torch.float32 else REL_TOL[psw_dtype], "grad_psw", cond=cp)
    assert (gp.cpu()[idx < 0] == 0).all()
    gW2, gp2 = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    assert torch.equal(gW, gW2) and torch.equal(gp, gp2)


# Unweighted bags (every weight 1) with hot rows: a bag holding a hot row k
# times merges to weight k; no psw-gradients (no dot product).
def test_backward_hot_rows_unweighted(device):
    from modelos_amd import embedding_bag as eb

    B, L, K, D = 1500, 10, 8000, 1024
    W, _, _, g = eb_inputs(B, L, K, D, torch.bfloat16, seed=63, psw=False)
    idx = _hot_matrix_indices(B, L, K, seed=64)
    gW, gp = eb.eb_backward(*_dev(idx, W, None, g, device=device))
    assert gp is None
    eW, _ = ref.eb_backward(idx, W, None, g)
    cW, _ = ref.eb_backward(idx, W.abs(), None, g.abs())
    assert_rel_close(gW, eW, REL_TOL[torch.bfloat16], "grad_weight", cond=cW)


# The merged weight of a hot row's bag is carried as bf16 hi + lo: sums that
# cancel down to the lo parts come out exact. Row 5: weight 1 + 2^-8 (float32
# weights; bf16 weights hold 1) in the even bags, -1 in the odd ones; row 6:
# held twice by the even bags (weights 1 and 2^-8, merged 1 + 2^-8), once by
# the odd ones (weight -1). Every partial sum is exact in float32, so the two
# rows' gradients are exact: 2 g (row 5: 0 for bf16 weights) and 2 g.
@pytest.mark.parametrize("psw_dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("D", [512, 1024])
def test_backward_hot_rows_merged_weights_exact(D, psw_dtype, device):
    from modelos_amd import embedding_bag as eb

    B, L, K = 1024, 4, 64
    gen = torch.Generator().manual_seed(61)
    W = (torch.randn((K, D), generator=gen) * 0.05).to(torch.bfloat16)
    idx = torch.randint(10, K, (B, L), generator=gen)
    p = torch.rand((B, L), generator=gen).to(psw_dtype)
    even = torch.arange(B) % 2 == 0
    w5 = 1 + 2.0**-8 if psw_dtype == torch.float32 else 1.0
    idx[:, 0] = 5
    p[:, 0] = torch.where(even, torch.tensor(w5), torch.tensor(-1.0)).to(psw_dtype)
    idx[:, 1] = 6
    p[:, 1] = torch.where(even, torch.tensor(1.0), torch.tensor(-1.0)).to(psw_dtype)
    idx[even, 2] = 6
    p[even, 2] = 2.0**-8
    col = torch.arange(D) % 3
    g = (1.0 + col).expand(B, D).to(torch.bfloat16).contiguous()  # 1, 2, 3 in every bag
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    gW = gW.cpu().float()
    want5 = (2.0 * (1.0 + col) if psw_dtype == torch.float32 else torch.zeros(D)).float()
    assert torch.equal(gW[5], want5)
    assert torch.equal(gW[6], (2.0 * (1.0 + col)).float())
    eW, ep = ref.eb_backward(idx, W, p, g)
    cW, cp = ref.eb_backward(idx, W.abs(), p.abs(), g.abs())
    assert_rel_close(gW, eW, REL_TOL[torch.bfloat16], "grad_weight", cond=cW)
    assert_rel_close(gp, ep, 1e-4 if psw_dtype == torch.float32 else REL_TOL[psw_dtype], "grad_psw", cond=cp)


# Rows longer than the row kernel's prefetch but below the heavy threshold
# (5..250 lookups), packed into the first 64-row windows, beside two heavy rows
# and uniform rows: with more than 3 lookups per row on average (the 8-slot
# prefetch) and fewer (4 slots; 2 for float32 rows of 1024).
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("K", [2000, 40000])
def test_backward_clustered_long_rows(K, dtype, device):
    from modelos_amd import embedding_bag as eb

    B, L, D = 512, 128, 1024
    g = torch.Generator().manual_seed(61)
    counts = torch.randint(5, 251, (200,), generator=g)
    ids = [torch.full((int(c),), r) for r, c in enumerate(counts)]
    ids += [torch.full((400,), 300), torch.full((1000,), 301)]
    ids = torch.cat(ids)
    rest = torch.randint(0, K, (B * L - ids.numel(),), generator=g)
    idx = torch.cat([ids, rest])[torch.randperm(B * L, generator=g)].view(B, L)
    W, _, p, gr = eb_inputs(B, L, K, D, dtype, seed=62)
    gW, gp = eb.eb_backward(*_dev(idx, W, p, gr, device=device))
    eW, ep = ref.eb_backward(idx, W, p, gr)
    cW, cp = ref.eb_backward(idx, W.abs(), p.abs(), gr.abs())
    assert_rel_close(gW, eW, REL_TOL[dtype], "grad_weight", cond=cW)
    assert_rel_close(gp, ep, REL_TOL[dtype], "grad_psw", cond=cp)
    gW2, gp2 = eb.eb_backward(*_dev(idx, W, p, gr, device=device))
    assert torch.equal(gW, gW2) and torch.equal(gp, gp2)


# Row counts past 2^20 change the sort's digit plan: 2 passes of 11-bit digits
# up to 2^22 rows, 3 passes of 10-bit digits beyond. Indices also sit on the
# digit boundaries and at the last row.
WIDE_K = [(700, 40, 3_000_000, 16), (300, 50, 5_000_000, 8)]


@pytest.mark.parametrize("B,L,K,D", WIDE_K, ids=lambda v: str(v))
def test_backward_wide_key_range(B, L, K, D, device):
    from modelos_amd import embedding_bag as eb

    dtype = torch.float32
    W, _, p, g = eb_inputs(B, L, K, D, dtype, seed=51 + D)
    idx = _hot_indices(B, L, K, seed=52 + D)
    edge = torch.tensor([0, 1, (1 << 10) - 1, 1 << 10, (1 << 11) - 1, 1 << 11, (1 << 20) - 1, 1 << 20,
                         (1 << 21) + 5, (1 << 22) - 1, K - 2, K - 1])
    edge = edge[edge < K]
    idx.view(-1)[-3 * edge.numel():] = edge.repeat(3)
    gW, gp = eb.eb_backward(*_dev(idx, W, p, g, device=device))
    eW, ep = ref.eb_backward(idx, W, p, g)
    cW, cp = ref.eb_backward(idx, W.abs(), p.abs(), g.abs())
    assert_rel_close(gW, eW, REL_TOL[dtype], "grad_weight", cond=cW)
    assert_rel_close(gp, ep, REL_TOL[dtype], "grad_psw", cond=cp)
    assert (gp.cpu()[idx < 0] == 0).all()


def test_backward_large_gradient_unweighted(device):
    from modelos_amd import embedding_bag as eb

    B, L, K, D = 4200, 8, 20000, 1024
    W, idx, _, g = eb_inputs(B, L, K, D, torch.bfloat16, seed=41, psw=False)
    gW, gp = eb.eb_backward(*_dev(idx, W, None, g, device=device))
    assert gp is None
    eW, _ = ref.eb_backward(idx, W, None, g)
    assert_rel_close(gW, eW, REL_TOL[torch.bfloat16], "unweighted grad_weight")


PREP_CASES = [
    (33, 17, 1000, 1024, torch.bfloat16, True),
    (9, 65, 300, 256, torch.float32, True),
    (5, 128, 2000, 2048, torch.float16, False),
    (17, 31, 100, 128, torch.bfloat16, True),
    (4, 2, 10, 32, torch.float32, True),
    (0, 8, 100, 512, torch.bfloat16, True),
    (512, 256, 70000, 1024, torch.bfloat16, True),
]


@pytest.mark.parametrize("B,L,K,D,dtype,weighted", PREP_CASES, ids=lambda v: str(v).replace("torch.", ""))
def test_backward_prepared_matches_direct(B, L, K, D, dtype, weighted, device):
    """pkm_eb_bwd_prepare on the side stream, then pkm_eb_bwd_prepared on the
    current one, gives pkm_eb_bwd's outputs bit for bit, out-of-range lookups
    (psw-gradient 0) included."""
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = eb_inputs(B, L, K, D, dtype, seed=41 + B)
    if B > 2:
        idx[1, 0] = -1
        idx[2, -1] = K + 5
    dW, didx, dp, dg = _dev(W, idx, p if weighted else None, g, device=device)
    gw0, gp0 = eb.eb_backward(didx, dW, dp, dg)
    prep = eb.eb_backward_prepare(didx, dW, dp)
    gw1, gp1 = eb.eb_backward(didx, dW, dp, dg, prepared=prep)
    torch.cuda.synchronize()
    assert torch.equal(gw0, gw1)
    if weighted:
        assert torch.equal(gp0, gp1)
        if B > 2:
            assert gp1[1, 0].item() == 0.0 and gp1[2, -1].item() == 0.0
    eW, ep = ref.eb_backward(idx, W, p if weighted else None, g)
    tol = REL_TOL[dtype]
    assert_rel_close(gw1, eW, tol, "prepared weight grad", cond=ref.eb_backward(idx, W.abs(), p.abs() if weighted else None, g.abs())[0])
    if weighted:
        assert_rel_close(gp1, ep, tol, "prepared psw grad")


def test_backward_prepared_rejects_other_lookups(device):
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = eb_inputs(8, 16, 500, 256, torch.bfloat16, seed=43)
    dW, didx, dp, dg = _dev(W, idx, p, g, device=device)
    prep = eb.eb_backward_prepare(didx, dW, dp)
    with pytest.raises(ValueError):
        eb.eb_backward(didx.clone(), dW, dp, dg, prepared=prep)


@pytest.mark.parametrize("K,hot", [(70000, False), (3000, False), (3000, True)])
def test_backward_prepared_workspace_serves_two_reductions(K, hot, device):
    """One prepared workspace, two reductions with different upstream
    gradients (retain_graph, or the same lookups reused): each reduction
    clears its own row-schedule counters, and leaves the hot-row lists the
    prepare built intact, so both equal pkm_eb_bwd's."""
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = eb_inputs(512, 256, K, 1024, torch.bfloat16, seed=47)
    if hot:
        idx = _hot_indices(512, 256, K, seed=49)  # rows 3, 4, 5 reach the hot threshold
    g2 = (torch.randn(g.shape, generator=torch.Generator().manual_seed(48)) * 0.5).to(g.dtype)
    dW, didx, dp, dg, dg2 = _dev(W, idx, p, g, g2, device=device)
    prep = eb.eb_backward_prepare(didx, dW, dp)
    gw1, gp1 = eb.eb_backward(didx, dW, dp, dg, prepared=prep)
    gw2, gp2 = eb.eb_backward(didx, dW, dp, dg2, prepared=prep)
    ew1, ep1 = eb.eb_backward(didx, dW, dp, dg)
    ew2, ep2 = eb.eb_backward(didx, dW, dp, dg2)
    torch.cuda.synchronize()
    assert torch.equal(gw1, ew1) and torch.equal(gp1, ep1)
    assert torch.equal(gw2, ew2) and torch.equal(gp2, ep2)


def test_backward_prepared_rejects_in_place_changes(device):
    """An in-place write to indices or psw after the prepare is refused (the
    workspace holds the sorted lookups and their weights)."""
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = eb_inputs(8, 16, 500, 256, torch.bfloat16, seed=44)
    dW, didx, dp, dg = _dev(W, idx, p, g, device=device)
    prep = eb.eb_backward_prepare(didx, dW, dp)
    dp.mul_(2.0)
    with pytest.raises(ValueError):
        eb.eb_backward(didx, dW, dp, dg, prepared=prep)
    prep = eb.eb_backward_prepare(didx, dW, dp)
    didx[0, 0] = 3
    with pytest.raises(ValueError):
        eb.eb_backward(didx, dW, dp, dg, prepared=prep)


# pkm_eb_bwd_accumulate: grad_weight + (the backward's table gradient), bit for
# bit the same as the backward into its own buffer followed by an add (what
# autograd forms for a table read twice), rows without lookups unchanged; on
# uniform lookups, hot rows (chunked partial sums) and clustered long rows
# (the long-row kernel). Shapes without an accumulating kernel return None.
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("pattern", ["uniform", "hot", "clustered"])
def test_backward_accumulate_equals_backward_plus_add(pattern, dtype, device):
    from modelos_amd import embedding_bag as eb

    B, L, K, D = 512, 64, 40000, 1024
    W, idx, p, gr = eb_inputs(B, L, K, D, dtype, seed=71)
    if pattern == "hot":
        idx = _hot_indices(B, L, K, seed=72)
    elif pattern == "clustered":
        g = torch.Generator().manual_seed(73)
        ids = torch.cat([torch.full((int(c),), r) for r, c in enumerate(torch.randint(5, 200, (60,), generator=g))])
        rest = torch.randint(0, K, (B * L - ids.numel(),), generator=g)
        idx = torch.cat([ids, rest])[torch.randperm(B * L, generator=g)].view(B, L)
    pending = torch.randn((K, D), generator=torch.Generator().manual_seed(74)).to(dtype)
    args = _dev(idx, W, p, gr, device=device)
    gW, gp = eb.eb_backward(*args)
    want = gW + pending.to(device)
    buf = pending.to(device)
    res = eb.eb_backward_into(*args, buf)
    assert res is not None
    got, gp2 = res
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want)
    assert torch.equal(gp2, gp)
    untouched = torch.ones(K, dtype=torch.bool)
    untouched[idx[idx >= 0].unique()] = False
    assert torch.equal(got.cpu()[untouched], pending[untouched])


def test_backward_accumulate_unsupported_returns_none(device):
    from modelos_amd import embedding_bag as eb

    B, L, K = 64, 16, 3000
    W, idx, p, gr = eb_inputs(B, L, K, 64, torch.float32, seed=75)  # 16 vectors a row: no 64-lane rows
    buf = torch.zeros((K, 64), device=device)
    assert eb.eb_backward_into(*_dev(idx, W, p, gr, device=device), buf) is None
    assert torch.count_nonzero(buf) == 0
    W, idx, p, gr = eb_inputs(B, L, K, 1024, torch.bfloat16, seed=76)
    idd, Wd, pd, gd = _dev(idx, W, p, gr, device=device)
    buf = torch.zeros((K, 1024), device=device, dtype=torch.bfloat16)
    assert eb.eb_backward_into(idd, Wd, pd, gd.float(), buf) is None  # float32 gradient of a bf16 table
    assert torch.count_nonzero(buf) == 0
