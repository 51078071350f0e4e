"""Host side of product-key retrieval: scores + per-half top-k + cartesian top-k.

`score_topk` runs the fused HIP kernel (pkm_score_topk) on torch's current
stream. `product_key_topk` wraps it in autograd:

  * the returned top-knn scores, and the optional full sub-score matrices
    s_1, s_2 (fast-weight PKM), are differentiable w.r.t. query and keys.
    For bfloat16 dot scores without sub-score gradients the backward is one
    call (pkm_score_grad_sparse): the nonzeros of each sub-score gradient row
    are listed and dq = dS @ K, dK = dS^T @ q run on MFMA from those lists.
    Otherwise it scatters the selected scores' gradient into dense sub-score
    gradients (pkm_score_grad_dense, deterministic, dense upstream gradients
    of s_1, s_2 added) and takes dq = dS @ K and dK = dS^T @ q as batched
    GEMMs per (head, half), as autograd does for the reference's einsum.

Reference: HashingMemory.get_indices (pkm/memory.py:250-289),
FastWeightProductKeyMemory.compute_qk_scores / get_indices
(fwpkm/fwpkm.py:853-934); autograd of einsum/cdist -> topk -> expand+add ->
topk -> gather there gives the same gradients.

There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib
from .embedding_bag import _aligned, _require_device

SCORE_TYPES = ("dot", "idw")


MAX_KNN = 1024
MAX_N_KEYS = 16384


def check_supported(n_keys: int, k_dim: int, knn: int, v_dim: int | None = None, what: str = "PKM layer") -> None:
    """Raises NotImplementedError, naming the limit, for sizes the HIP kernels
    have no path for:
      retrieval (pkm_score_topk): 1 <= knn <= min(n_keys, 1024), n_keys up to
        16384, any even k_dim (the tuned kernels take knn <= 64, n_keys a
        multiple of 64 up to 2048 and k_dim / 2 a multiple of 16 / 32 in
        float32 / bfloat16; the other shapes and float16 run on the generic
        kernel);
      value bag backward (pkm_eb_bwd): v_dim a power of two from 4 to 4096
        (2048 for float32), as the reference's Triton kernels need a power of
        two (pkm/xformer_embeddingbag.py:97-113, 291-328)."""
    problems = []
    if not 1 <= knn <= MAX_KNN:
        problems.append(f"knn={knn} (must be 1..{MAX_KNN})")
    if not 1 <= n_keys <= MAX_N_KEYS:
        problems.append(f"n_keys={n_keys} (must be 1..{MAX_N_KEYS})")
    if knn > n_keys:
        problems.append(f"knn={knn} > n_keys={n_keys}")
    if k_dim < 2 or k_dim % 2:
        problems.append(f"k_dim={k_dim} (must be even)")
    if v_dim is not None and (v_dim < 4 or v_dim > 4096 or v_dim & (v_dim - 1)):
        problems.append(f"value dim={v_dim} (must be a power of two from 4 to 4096)")
    if problems:
        raise NotImplementedError(f"{what}: the MI355X HIP kernels do not support " + ", ".join(problems))


def _check(query: torch.Tensor, keys: torch.Tensor, heads: int, knn: int, score_type: str):
    if score_type not in SCORE_TYPES:
        raise ValueError(f"score_type must be one of {SCORE_TYPES}, got {score_type!r}")
    if keys.dim() != 2:
        raise ValueError(f"keys must be [2 * heads * n_keys, k_dim // 2], got shape {tuple(keys.shape)}")
    half = keys.shape[1]
    k_dim = 2 * half
    if query.shape[-1] != k_dim:
        raise ValueError(f"query last dim {query.shape[-1]} != 2 * keys.shape[1] = {k_dim}")
    if query.numel() % (heads * k_dim) != 0:
        raise ValueError(f"query of shape {tuple(query.shape)} is not [tokens, {heads}, {k_dim}]")
    if keys.shape[0] % (2 * heads) != 0:
        raise ValueError(f"keys rows {keys.shape[0]} not a multiple of 2 * heads = {2 * heads}")
    if query.dtype != keys.dtype:
        raise TypeError(f"query dtype {query.dtype} != keys dtype {keys.dtype}")
    n = keys.shape[0] // (2 * heads)
    if not 1 <= knn <= n:
        raise ValueError(f"knn must be in [1, n_keys={n}], got {knn}")
    return query.numel() // (heads * k_dim), n, half


def score_topk(
    query: torch.Tensor,
    keys: torch.Tensor,
    heads: int,
    knn: int,
    score_type: str = "dot",
    sub_outputs: bool = False,
):
    """Forward only (no autograd).

    query: [tokens, heads, k_dim] (or any view with that many elements, e.g.
    [tokens * heads, k_dim]); keys: [2 * heads * n_keys, k_dim // 2].
    Returns scores, indices [tokens * heads, knn] and, with sub_outputs,
    additionally i1, i2 [tokens, heads, knn] and s1, s2 [tokens, heads, n_keys].
    """
    N, n, half = _check(query, keys, heads, knn, score_type)
    dev = _require_device(query, keys)
    query = _aligned(query)
    keys = _aligned(keys)
    dt = query.dtype
    scores = torch.empty((N * heads, knn), dtype=dt, device=dev)
    indices = torch.empty((N * heads, knn), dtype=torch.long, device=dev)
    i1 = i2 = s1 = s2 = None
    if sub_outputs:
        i1 = torch.empty((N, heads, knn), dtype=torch.long, device=dev)
        i2 = torch.empty((N, heads, knn), dtype=torch.long, device=dev)
        s1 = torch.empty((N, heads, n), dtype=dt, device=dev)
        s2 = torch.empty((N, heads, n), dtype=dt, device=dev)
    # workspace for the keys packed tile-major (taken by the tile kernel only)
    ws = torch.empty(keys.numel() * keys.element_size(), dtype=torch.uint8, device=dev)
    _lib.call(
        "pkm_score_topk_ws",
        _lib.ptr(query), _lib.ptr(keys), N, heads, n, half, knn,
        _lib.SCORE_CODES[score_type], _lib.dtype_code(query),
        _lib.ptr(scores), _lib.ptr(indices), _lib.ptr(i1), _lib.ptr(i2), _lib.ptr(s1), _lib.ptr(s2),
        _lib.ptr(ws), ws.numel(), _lib.stream_of(dev),
    )
    if sub_outputs:
        return scores, indices, i1, i2, s1, s2
    return scores, indices


def score_grad_dense(indices: torch.Tensor, d_scores: torch.Tensor, heads: int, n_keys: int,
                     d_sub1: torch.Tensor | None = None, d_sub2: torch.Tensor | None = None) -> torch.Tensor:
    """Dense gradient of the sub-score matrices, [heads, 2, tokens, n_keys] in
    d_scores.dtype, from the gradient of the selected scores (and optional
    dense upstream gradients of s1, s2 [tokens, heads, n_keys])."""
    dev = _require_device(indices, d_scores, d_sub1, d_sub2)
    NH, knn = indices.shape
    N = NH // heads
    dt = d_scores.dtype
    d_sub1 = _aligned(d_sub1.to(dt)) if d_sub1 is not None else None
    d_sub2 = _aligned(d_sub2.to(dt)) if d_sub2 is not None else None
    dS = torch.empty((heads, 2, N, n_keys), dtype=dt, device=dev)
    _lib.call(
        "pkm_score_grad_dense",
        _lib.ptr(indices.contiguous()), _lib.ptr(d_scores.contiguous()), _lib.dtype_code(d_scores),
        N, heads, n_keys, knn, _lib.ptr(d_sub1), _lib.ptr(d_sub2), _lib.ptr(dS), _lib.stream_of(dev),
    )
    return dS


def score_grad_sparse(query: torch.Tensor, keys: torch.Tensor, indices: torch.Tensor, d_scores: torch.Tensor,
                      heads: int, need_query: bool = True, need_keys: bool = True):
    """Gradients (d_query [tokens, heads, k_dim], d_keys like keys; None where
    not needed) of the selected dot-product scores, from the sparse rows of
    the sub-score gradient on MFMA (pkm_score_grad_sparse): bfloat16 only.
    Returns None when these sizes are outside the kernel's limits."""
    dev = _require_device(query, keys, indices, d_scores)
    half = keys.shape[1]
    n = keys.shape[0] // (2 * heads)
    NH, knn = indices.shape
    N = NH // heads
    if query.dtype != torch.bfloat16 or keys.dtype != torch.bfloat16:
        return None
    ws_bytes = int(_lib.load().pkm_score_grad_sparse_workspace_size(N, heads, n, half, knn))
    if ws_bytes == 0:
        return None
    query = _aligned(query)
    keys = _aligned(keys)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    dq = torch.empty((N, heads, 2 * half), dtype=query.dtype, device=dev) if need_query else None
    dk = torch.empty_like(keys) if need_keys else None
    _lib.call(
        "pkm_score_grad_sparse",
        _lib.ptr(indices.contiguous()), _lib.ptr(d_scores.to(query.dtype).contiguous()), _lib.dtype_code(query),
        N, heads, n, half, knn, _lib.ptr(query), _lib.ptr(keys), _lib.ptr(dq), _lib.ptr(dk),
        _lib.ptr(ws), ws_bytes, _lib.stream_of(dev),
    )
    return dq, dk


class _DenseScoreGrad(torch.autograd.Function):
    """score_grad_dense as an autograd node (a scatter-add of the selected
    scores' gradient plus the dense sub-score gradients), so that a backward
    taken with create_graph (the fast-weight inner step) stays
    differentiable. Its VJP is the matching gather."""

    @staticmethod
    def forward(ctx, indices, d_scores, d_sub1, d_sub2, heads, n_keys):
        ctx.save_for_backward(indices)
        ctx.heads, ctx.n = heads, n_keys
        ctx.has_sub = (d_sub1 is not None, d_sub2 is not None)
        return score_grad_dense(indices, d_scores, heads, n_keys, d_sub1, d_sub2)

    @staticmethod
    def backward(ctx, g):
        (indices,) = ctx.saved_tensors
        H, n = ctx.heads, ctx.n
        NH, knn = indices.shape
        N = NH // H
        idx = indices.view(N, H, knn)
        g0 = g[:, 0].permute(1, 0, 2)  # [N, H, n]
        g1 = g[:, 1].permute(1, 0, 2)
        d_scores = (g0.gather(2, idx // n) + g1.gather(2, idx % n)).reshape(NH, knn)
        return (None, d_scores, g0 if ctx.has_sub[0] else None, g1 if ctx.has_sub[1] else None, None, None)


IDW_COEF_MAX_N = 1024  # pkm_idw_grad_coef's n_keys limit


def _idw_grad_coef(dS, qq, kk, dots):
    """(U, rowsum, colsum) of pkm_idw_grad_coef: U = dS / (1e-3 + d2) where
    d2 = (qq + kk) - 2 dots > 0, else 0, float32 [batches, tokens, n]."""
    B, T, n = dots.shape
    dS = dS.contiguous()
    qq, kk, dots = qq.float().contiguous(), kk.float().contiguous(), dots.contiguous()
    dev = dots.device
    U = torch.empty((B, T, n), device=dev, dtype=torch.float32)
    rs = torch.empty((B, T), device=dev, dtype=torch.float32)
    cs = torch.empty((B, n), device=dev, dtype=torch.float32)
    ws_bytes = int(_lib.load().pkm_idw_grad_coef_workspace_size(B, T, n))
    ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    _lib.call("pkm_idw_grad_coef", _lib.ptr(dS), _lib.dtype_code(dS), _lib.ptr(qq), _lib.ptr(kk), _lib.ptr(dots), B, T,
              n, _lib.ptr(U), _lib.ptr(rs), _lib.ptr(cs), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev))
    return U, rs, cs


def share_distance_products(sub_scores: torch.Tensor, dots: torch.Tensor, qq: torch.Tensor, kk: torch.Tensor) -> None:
    """Hands the float32 distance operands of an idw retrieval (dots [2 heads,
    tokens, n] = <q_t, k_j>, qq [2 heads, tokens], kk [2 heads, n], taken from
    the retrieval's own query and forward-time keys) to its backward node,
    found through one of its sub-score outputs, so that the backward does not
    form them again. No effect for other outputs or score types."""
    node = sub_scores.grad_fn
    if node is not None and getattr(node, "score_type", None) == "idw" and getattr(node, "sub_outputs", False):
        node.shared_products = (dots, qq, kk)


def _grads_from_dense(query, keys, dS, heads, n, score_type, keys_fwd=None, shared=None):
    """dq [tokens, heads, k_dim] and dkeys [2*heads*n, half] from the dense
    sub-score gradient dS [heads, 2, tokens, n] with one pair of batched GEMMs
    per (head, half) — the products autograd forms for the reference's einsum
    (dot) or cdist (idw) on the full score matrices. Torch ops: differentiable
    when the backward runs with create_graph.

    Which key values the products read follows the reference's saved tensors
    (the fast-weight module stores updated weights into the key table in
    place after its forward, fwpkm.py:540-545, so a table saved by reference
    is read as it is at backward time): the einsum (dot) saves the key table
    itself; cdist with use_mm_for_euclid_dist (idw) on the table's
    strided half view works on a copy made at forward time, so every value
    it reads, first and second order, is the forward-time one. `keys_fwd` is
    that copy (idw); under create_graph it carries the table's own autograd
    identity. `shared`: (dots, qq, kk) already formed from the same query and
    forward-time keys (share_distance_products), used outside create_graph."""
    half = keys.shape[1]
    N = dS.shape[2]
    Kh = keys.reshape(heads * 2, n, half)
    qh = query.reshape(N, heads, 2, half).permute(1, 2, 0, 3).reshape(heads * 2, N, half)
    D = dS.view(heads * 2, N, n)
    if score_type == "dot":
        dqh = torch.bmm(D, Kh)  # [2H, N, half]
        dk = torch.bmm(D.transpose(1, 2), qh)  # [2H, n, half]
    else:
        # s = -log(1e-3 + d^2), d^2 = |q|^2 + |k|^2 - 2<q,k> (0 where not positive):
        #   ds/dq = 2 u (k - q), ds/dk = 2 u (q - k), u = 1 / (1e-3 + d^2)
        q32, k32 = qh.float(), Kh.float()
        kf = k32
        if keys_fwd is not None:
            # the forward-time values; under create_graph differentiable as the table itself
            kf = keys_fwd.reshape(heads * 2, n, half).float()
            if torch.is_grad_enabled():
                kf = kf + (k32 - k32.detach())
        use_shared = shared is not None and not torch.is_grad_enabled()
        dots = shared[0] if use_shared else torch.bmm(q32, kf.transpose(1, 2).contiguous())
        if torch.is_grad_enabled() or n > IDW_COEF_MAX_N:
            # differentiable in turn (a backward taken with create_graph), or more keys than the kernel takes
            d2 = (q32 * q32).sum(-1)[:, :, None] + (kf * kf).sum(-1)[:, None, :] - 2.0 * dots
            U = torch.where(d2 > 0, D.float() / (1e-3 + d2.clamp_min(0.0)), torch.zeros_like(d2))
            rs, cs = U.sum(-1), U.sum(1)
        else:
            # the same U and its row and column sums in one pass (pkm_idw_grad_coef)
            qq, kk = (shared[1], shared[2]) if use_shared else ((q32 * q32).sum(-1), (kf * kf).sum(-1))
            U, rs, cs = _idw_grad_coef(D, qq, kk, dots)
        dqh = 2.0 * (torch.bmm(U, kf) - q32 * rs[:, :, None])
        # float32 operands: the transposed view goes to the GEMM as it is
        dk = 2.0 * (torch.bmm(U.transpose(1, 2), q32) - kf * cs[:, :, None])
    dq = dqh.view(heads, 2, N, half).permute(2, 0, 1, 3).reshape(N, heads, 2 * half)
    return dq, dk.reshape(keys.shape)


class ProductKeyTopK(torch.autograd.Function):
    """Differentiable product-key retrieval (scores w.r.t. query and keys)."""

    @staticmethod
    def forward(ctx, query, keys, heads, knn, score_type, sub_outputs):
        ctx.set_materialize_grads(False)  # no zero tensors for the outputs without a gradient
        outs = score_topk(query, keys, heads, knn, score_type, sub_outputs)
        ctx.heads, ctx.knn, ctx.score_type, ctx.sub_outputs = heads, knn, score_type, sub_outputs
        ctx.n = keys.shape[0] // (2 * heads)
        ctx.query_shape = query.shape
        # idw: the key values the distances were taken at (see _grads_from_dense)
        saved = (query, keys, outs[1]) + ((keys.detach().clone(),) if score_type == "idw" else ())
        ctx.save_for_backward(*saved)
        ctx.mark_non_differentiable(*(outs[1:4] if sub_outputs else outs[1:2]))
        return outs

    @staticmethod
    def backward(ctx, d_scores, d_indices, *rest):
        query, keys, indices = ctx.saved_tensors[:3]
        keys_fwd = ctx.saved_tensors[3] if ctx.score_type == "idw" else None
        heads, n = ctx.heads, ctx.n
        d_s1 = rest[2] if ctx.sub_outputs else None
        d_s2 = rest[3] if ctx.sub_outputs else None
        if d_scores is None:
            d_scores = torch.zeros(indices.shape, dtype=query.dtype, device=query.device)
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grads = None
        # the sparse kernel's gradients are not differentiable: a create_graph backward takes the dense path
        if ctx.score_type == "dot" and d_s1 is None and d_s2 is None and not torch.is_grad_enabled():
            grads = score_grad_sparse(query, keys, indices, d_scores, heads, need_q, need_k)
        if grads is not None:
            dq, dk = grads
        else:
            d_s1 = d_s1.to(query.dtype) if d_s1 is not None else None
            d_s2 = d_s2.to(query.dtype) if d_s2 is not None else None
            dS = _DenseScoreGrad.apply(indices, d_scores.to(query.dtype), d_s1, d_s2, heads, n)
            dq, dk = _grads_from_dense(query, keys, dS, heads, n, ctx.score_type, keys_fwd,
                                       getattr(ctx, "shared_products", None))
        d_query = dq.to(query.dtype).reshape(ctx.query_shape) if ctx.needs_input_grad[0] else None
        d_keys = dk.to(keys.dtype) if ctx.needs_input_grad[1] else None
        return d_query, d_keys, None, None, None, None


class _ScoreSoftmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        x2 = _aligned(x)
        rows, cols = x2.shape
        y = torch.empty_like(x2)
        _lib.call("pkm_softmax_fwd", _lib.ptr(x2), rows, cols, _lib.dtype_code(x2), _lib.ptr(y),
                  _lib.stream_of(x2.device))
        # the input itself: a create_graph backward differentiates through it
        # (an aligned copy made here, with grad off, would cut that path)
        ctx.save_for_backward(x)
        return y

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        if torch.is_grad_enabled():
            # a create_graph backward (the fast-weight inner step): the same float32 expression in
            # torch ops, so that it is differentiable in turn
            p = torch.softmax(x.float(), dim=-1)
            dyf = dy.float()
            return (p * (dyf - (dyf * p).sum(-1, keepdim=True))).to(x.dtype)
        x2 = _aligned(x)
        rows, cols = x2.shape
        dy2 = _aligned(dy.to(x2.dtype))
        dx = torch.empty_like(x2)
        _lib.call("pkm_softmax_bwd", _lib.ptr(dy2), _lib.ptr(x2), rows, cols, _lib.dtype_code(x2), _lib.ptr(dx),
                  _lib.stream_of(x2.device))
        return dx


_SOFTMAX_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def score_softmax(scores: torch.Tensor) -> torch.Tensor:
    """F.softmax(scores.float(), dim=-1).type_as(scores) (pkm/memory.py:218)
    with one kernel each way (pkm_softmax_fwd / pkm_softmax_bwd): float32,
    bfloat16 or float16 rows of 1 to 65536 scores. Other dtypes raise."""
    _require_device(scores)
    k = scores.shape[-1]
    if scores.dtype not in _SOFTMAX_DTYPES:
        raise NotImplementedError(f"score_softmax: dtype {scores.dtype} not supported (float32, bfloat16, float16 are)")
    if k == 0:
        return torch.empty_like(scores)
    return _ScoreSoftmax.apply(scores.reshape(-1, k)).view(scores.shape)


def product_key_topk(
    query: torch.Tensor,
    keys: torch.Tensor,
    heads: int,
    knn: int,
    score_type: str = "dot",
    sub_outputs: bool = False,
) -> Tuple[torch.Tensor, ...]:
    """Autograd version of score_topk (same arguments and outputs)."""
    return ProductKeyTopK.apply(query, keys, heads, knn, score_type, sub_outputs)


__all__ = ["check_supported", "score_topk", "product_key_topk", "ProductKeyTopK", "score_grad_dense", "score_grad_sparse", "score_softmax",
           "SCORE_TYPES"]
