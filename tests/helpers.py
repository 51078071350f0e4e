"""Shared input generators and comparison helpers for the tests."""
from __future__ import annotations

import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def eb_inputs(B, L, K, D, dtype, seed=0, psw=True, psw_dtype=None, softmax=True, with_grad=True, scale=None):
    """Seeded CPU inputs for an embedding-bag case, drawn in a fixed order:
    weight, indices, psw, grad."""
    g = gen(seed)
    scale = (D**-0.5) if scale is None else scale
    W = (torch.randn((K, D), generator=g) * scale).to(dtype)
    idx = torch.randint(0, max(K, 1), (B, L), generator=g, dtype=torch.long)
    p = None
    if psw:
        logits = torch.randn((B, L), generator=g)
        p = (torch.softmax(logits, -1) if softmax else logits).to(psw_dtype or dtype)
    grad = torch.randn((B, D), generator=g).to(dtype) if with_grad else None
    return W, idx, p, grad


REL_TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float64: 1e-12}


def assert_rel_close(actual: torch.Tensor, expected: torch.Tensor, rel: float, what: str = "", atol: float = 0.0,
                     elem_frac: float | None = 0.1, cond: torch.Tensor | None = None):
    """Two bounds, both enforced on every element:
      normwise:    |a - e| <= rel * |e| + rel * max|e| + atol (relative error
                   with an absolute floor at the tensor's scale, for sums with
                   cancellation; atol covers tensors that are zero up to rounding);
      elementwise: |a - e| <= rel * |e| + atol wherever |e| >= elem_frac * max|e|
                   (pure relative error of the elements that carry the tensor's
                   magnitude; elem_frac=None skips it), or, when `cond` is given
                   (the same sums taken over the terms' absolute values, so
                   cond >= |e|), |a - e| <= rel * cond + atol on every element:
                   the rounding-error bound of a sum, which stays meaningful for
                   elements that are small through cancellation.
    """
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    scale = e.abs().max().item() if e.numel() else 0.0
    err = (a - e).abs()
    bound = rel * e.abs() + rel * scale + atol + 1e-30
    bad = err > bound
    kind = "normwise"
    if not bad.any() and cond is not None:
        c = cond.detach().to("cpu", torch.float64)
        assert c.shape == e.shape, f"{what}: cond shape {tuple(c.shape)} != {tuple(e.shape)}"
        bad = err > rel * c + atol + 1e-30
        kind = "elementwise (rel * sum of |terms|)"
    elif not bad.any() and elem_frac is not None:
        big = e.abs() >= elem_frac * scale
        bad = big & (err > rel * e.abs() + atol + 1e-30)
        kind = f"elementwise (|e| >= {elem_frac} * max|e|)"
    if bad.any():
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} / {a.numel()} elements off the {kind} bound; first at flat {i}: "
            f"got {a.reshape(-1)[i].item()!r} expected {e.reshape(-1)[i].item()!r} "
            f"(max abs err {err.max().item():.3e}, scale {scale:.3e}, rel {rel})"
        )


def assert_norm_close(actual: torch.Tensor, expected: torch.Tensor, rel: float, what: str = ""):
    """Normwise relative error in the 2-norm, ||a - e|| <= rel * ||e||: for
    long chains of rounded stages whose outputs are sums with heavy
    cancellation, where single elements can carry the input rounding of many
    terms beyond their own size."""
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    err = (a - e).norm().item()
    ref = e.norm().item()
    assert err <= rel * ref, f"{what}: ||a - e|| = {err:.3e} > {rel} * ||e|| = {rel * ref:.3e}"

