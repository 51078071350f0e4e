"""Drop-in for the reference's fwpkm/fwpkm.py: the fast-weight product-key memory.

FastWeightProductKeyMemory keeps the reference's constructor arguments,
parameter names and shapes (`keys` [2 * heads * n_subkeys, k_dim / 2],
`values` [n_subkeys^2, v_dim]), its methods and their return conventions
(fwpkm.py:22-934), so modeling code calls it unchanged. The in-context
update runs on gfx950 HIP kernels:

  * get_indices: sub-key scores (dot product or idw), per-half top-k and the
    cartesian top-k in one fused kernel, which also writes the full sub-score
    matrices the marginal-entropy address loss reads; differentiable w.r.t.
    query and keys, including through those matrices (product_keys);
  * score_transform: the softmax over heads x top-k on one kernel each way;
  * retrieve_values: the weighted bag over the fast values (forward gather,
    deterministic first-order backward, and the fused double backward the
    outer loss takes through the inner gradient step);
  * update_fw: the values' SGD step (sample-count scaling, division by the
    slot access counts, optional clipping, weight decay) in one pass over the
    table, differentiable for the outer loss;
  * the marginal-entropy address loss and the keys' gradient of it, with its
    own double backward (marginal_entropy), over the top-k entries of each
    sub-score row.

The mean squared error and the chunk loop are torch code around these
kernels, with the reference's
semantics, including its quirks: the output of a chunk is read before that
chunk's update; the streaming path normalises the update with the forward
chunk's indices and counts samples as B * chunk length; addr_loss=None with
mem_grad_to_values_only=True fails in the keys' update (fwpkm.py:266-272,
298-318).

There is no CPU path: the kernels raise on CPU tensors.
"""
from __future__ import annotations

from collections import OrderedDict, defaultdict
from logging import getLogger
import math
from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from .. import _lib
from ..embedding_bag import _aligned, _require_device
from ..product_keys import check_supported, product_key_topk, score_softmax
from .marginal_entropy import addr_loss_and_key_grad, supported as _me_supported
from .xformer_embeddingbag_grad_wrapper import xformers_embedding_bag

logger = getLogger()

SCORE_TYPES = {"dot_product": "dot", "idw": "idw"}


def l2norm(x: torch.FloatTensor, dim: int = -1, eps: float = 1e-6):
    """x / sqrt(sum(x^2) + eps) along `dim` (fwpkm.py:16-19; the FLA library's l2norm)."""
    return x * torch.rsqrt((x * x).sum(dim=dim, keepdim=True) + eps)


def _score_type(name: str) -> str:
    try:
        return SCORE_TYPES[name]
    except KeyError:
        raise NotImplementedError(f"QK score type {name} not implemented.") from None


def get_indices(query: torch.Tensor, keys: torch.Tensor, heads: int, k_dim: int, topk: int,
                qk_score_type: str = "dot_product"):
    """fwpkm.py:871-934 as a function. query: [BT, heads, k_dim] (any view with
    that many elements); keys: [heads * 2 * subsize, k_dim // 2].
    Returns scores, indices, topk_indices1, topk_indices2 [BT, heads, topk] and
    scores1, scores2 [BT, heads, subsize]; equal scores are ordered by the
    smaller sub-key position."""
    BT = query.numel() // (heads * k_dim)
    q = query.reshape(BT, heads, k_dim)
    scores, idx, i1, i2, s1, s2 = product_key_topk(q, keys, heads, topk, _score_type(qk_score_type),
                                                   sub_outputs=True)
    return (scores.view(BT, heads, topk), idx.view(BT, heads, topk), i1, i2, s1, s2)


def compute_qk_scores(q: torch.Tensor, k: torch.Tensor, qk_score_type: str = "dot_product") -> torch.Tensor:
    """fwpkm.py:853-869: q [batch, heads, d], k [heads, n_keys, d] -> scores
    [batch, heads, n_keys] (dot product, or -log(1e-3 + squared distance)).
    Dense scores without selection are a plain batched GEMM; this form exists
    for callers of the method itself — get_indices never materialises it
    apart from the sub-score outputs."""
    st = _score_type(qk_score_type)
    _require_device(q, k)
    qh = q.permute(1, 0, 2).contiguous()  # [heads, batch, d]
    dots = torch.bmm(qh, k.transpose(1, 2).contiguous())  # [heads, batch, n_keys]
    if st == "dot":
        return dots.permute(1, 0, 2)
    d2 = (qh * qh).sum(-1, keepdim=True) + (k * k).sum(-1)[:, None, :] - 2.0 * dots
    return (-torch.log(1e-3 + d2.clamp_min(0.0))).permute(1, 0, 2)


class _SgdValueUpdate(torch.autograd.Function):
    """(new values, scaled gradient) of the values' SGD step (pkm_fw_sgd_update)."""

    @staticmethod
    def forward(ctx, p, g, counts, scale, lr, wd, clip):
        p2 = _aligned(p)
        g2 = _aligned(g.to(p.dtype))
        counts = counts.contiguous()
        new = torch.empty_like(p2)
        gs = torch.empty_like(p2)
        K, D = p2.shape
        _lib.call("pkm_fw_sgd_update", _lib.ptr(p2), _lib.ptr(g2), _lib.ptr(counts), K, D, _lib.dtype_code(p2),
                  float(scale), float(lr), float(wd), int(bool(clip)), _lib.ptr(gs), _lib.ptr(new),
                  _lib.stream_of(p2.device))
        ctx.save_for_backward(gs, counts)
        ctx.scale, ctx.lr, ctx.wd, ctx.clip = scale, lr, wd, clip
        # an output no loss reaches gets None, not a [K, D] tensor of zeros
        ctx.set_materialize_grads(False)
        return new, gs

    @staticmethod
    def backward(ctx, d_new, d_gs):
        # the reference's autograd through p - lr * (clamp(g * scale / c) + wd * p), op by op
        # (pkm_fw_sgd_update_bwd); only the scaled gradient's own gradient: its two ops
        gs, counts = ctx.saved_tensors
        if d_new is None:
            if d_gs is None or not ctx.needs_input_grad[1]:
                return None, None, None, None, None, None, None
            c = counts.to(gs.dtype)
            c[c == 0] = 1.0
            return None, (d_gs / c.unsqueeze(-1)) * ctx.scale, None, None, None, None, None
        dn = _aligned(d_new.to(gs.dtype))
        dgi = _aligned(d_gs.to(gs.dtype)) if d_gs is not None else None
        d_p = torch.empty_like(gs)
        d_g = torch.empty_like(gs)
        K, D = gs.shape
        _lib.call("pkm_fw_sgd_update_bwd", _lib.ptr(dn), _lib.ptr(dgi), _lib.ptr(gs), _lib.ptr(counts), K, D,
                  _lib.dtype_code(gs), float(ctx.scale), float(ctx.lr), float(ctx.wd), int(bool(ctx.clip)),
                  _lib.ptr(d_p), _lib.ptr(d_g), _lib.stream_of(gs.device))
        return (d_p if ctx.needs_input_grad[0] else None), (d_g if ctx.needs_input_grad[1] else None), \
            None, None, None, None, None


class _GradSink:
    """A table gradient parked by one consumer's backward for another's to
    add its own into (_TableFanout)."""

    __slots__ = ("pending",)

    def __init__(self):
        self.pending = None

    def take(self):
        p, self.pending = self.pending, None
        return p


class _TableFanout(torch.autograd.Function):
    """Two handles on one fast-weight table, its chunk's retrieval's and its
    update step's. Their gradients meet in a sink: the step's backward parks
    its table gradient there and the retrieval's bag backward adds its own
    into it in place (pkm_eb_bwd_accumulate), instead of autograd adding two
    dense [K, D] gradients in a pass of its own. Whatever is still parked or
    arrives separately is added here (any order of the two backward passes)."""

    @staticmethod
    def forward(ctx, table, sink):
        ctx.sink = sink
        ctx.set_materialize_grads(False)  # a handle without a gradient arrives as None, not a [K, D] of zeros
        return table.view_as(table), table.view_as(table)

    @staticmethod
    def backward(ctx, g_read, g_step):
        parts = [g for g in (g_read, g_step, ctx.sink.take()) if g is not None]
        if not parts:
            return None, None
        out = parts[0]
        for g in parts[1:]:
            out = out + g
        return out, None


def _fan_out(table: torch.Tensor):
    """(handle for the retrieval, handle for the update step) of `table`."""
    sink = _GradSink()
    read, step = _TableFanout.apply(table, sink)
    read._pkm_grad_sink = sink
    step._pkm_grad_sink = sink
    return read, step


class _FusedValueStep(torch.autograd.Function):
    """FwPKM's values step taken straight from the gradient of the memory loss
    w.r.t. the bag output: the table gradient EB^T(indices, psw, d_hyp) and the
    bincount-normalised SGD step in one pass over the table (pkm_eb_bwd_sgd).
    Returns (new values, scaled gradient, per-row sums of its squares); with
    want_scaled False the scaled gradient is None (not written) unless the
    backward of a clipped or weight-decayed step needs it.

    Its backward is the reference's through EmbeddingBagBW and the step
    (fwpkm/xformer_embeddingbag_grad_wrapper.py:42-74, fwpkm.py:351-365):
    the values get d_new (plus the weight decay's term); d_hyp and psw get the
    double backward of the bag over the gradient of the table gradient, which
    pkm_eb_bwd2_sgd forms row by row as it gathers (never a dense [K, D])."""

    @staticmethod
    def forward(ctx, values, indices, psw, d_hyp, scale, lr, wd, clip, want_scaled=True):
        from ..embedding_bag import eb_backward_workspace_bytes

        V = _aligned(values)
        idx = indices.contiguous()
        w = psw.contiguous()
        g = _aligned(d_hyp.to(V.dtype))
        K, D = V.shape
        B, L = idx.shape
        new = torch.empty_like(V)
        # the scaled gradient: when asked for, or when the backward of a clipped or weight-decayed
        # step reads it (otherwise None, and no [K, D] write)
        gs = torch.empty_like(V) if (want_scaled or clip or wd != 0.0) else None
        counts = torch.empty(K, dtype=torch.int32, device=V.device)
        sumsq = torch.empty(K, dtype=torch.float32, device=V.device)
        ws_bytes = eb_backward_workspace_bytes(K, D, B, L)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=V.device)
        _lib.call("pkm_eb_bwd_sgd", _lib.ptr(V), K, D, _lib.dtype_code(V), _lib.ptr(idx), _lib.ptr(w),
                  _lib.dtype_code(w), _lib.ptr(g), B, L, float(scale), float(lr), float(wd), int(bool(clip)),
                  _lib.ptr(new), _lib.ptr(gs), None, _lib.ptr(counts), _lib.ptr(sumsq), _lib.ptr(ws), ws_bytes,
                  _lib.stream_of(V.device))
        ctx.save_for_backward(gs, counts, idx, w, g)
        ctx.scale, ctx.lr, ctx.wd, ctx.clip = scale, lr, wd, clip
        ctx.table = (K, D, V.dtype)
        ctx.sink = getattr(values, "_pkm_grad_sink", None)
        ctx.mark_non_differentiable(sumsq)
        # the scaled gradient usually reaches no loss: None, not a [K, D] of zeros
        # (which the double backward would also read)
        ctx.set_materialize_grads(False)
        return new, gs, sumsq

    @staticmethod
    def backward(ctx, d_new, d_gs, _d_sumsq):
        gs, counts, idx, w, g = ctx.saved_tensors
        if d_new is None and d_gs is None:
            return (None,) * 9
        K, D, dt = ctx.table
        B, L = idx.shape
        dn = _aligned(d_new.to(dt)) if d_new is not None else torch.zeros((K, D), dtype=dt, device=idx.device)
        dgi = _aligned(d_gs.to(dt)) if d_gs is not None else None
        d_values = None
        if ctx.needs_input_grad[0]:
            if ctx.wd == 0.0:
                d_values = dn  # p - lr * (step + 0 * p): the identity path alone
            else:
                d_values = torch.empty_like(dn)
                cnt64 = counts.to(torch.int64)
                _lib.call("pkm_fw_sgd_update_bwd", _lib.ptr(dn), None, _lib.ptr(gs), _lib.ptr(cnt64), K, D,
                          _lib.dtype_code(gs), float(ctx.scale), float(ctx.lr), float(ctx.wd), int(bool(ctx.clip)),
                          _lib.ptr(d_values), None, _lib.stream_of(gs.device))
        d_hyp = d_psw = None
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            d_hyp = torch.empty((B, D), dtype=dt, device=dn.device)
            d_psw = torch.empty_like(w)
            _lib.call("pkm_eb_bwd2_sgd", _lib.ptr(dn), _lib.ptr(dgi), _lib.ptr(gs), _lib.ptr(counts), K, D,
                      _lib.dtype_code(dn), float(ctx.scale), float(ctx.lr), int(bool(ctx.clip)), _lib.ptr(idx),
                      _lib.ptr(w), _lib.dtype_code(w), _lib.ptr(g), B, L, _lib.ptr(d_hyp), _lib.ptr(d_psw),
                      _lib.stream_of(dn.device))
        if d_values is not None and ctx.sink is not None and not torch.is_grad_enabled():
            # parked for the retrieval's bag backward to add its gradient into (_TableFanout)
            ctx.sink.pending = d_values if ctx.sink.pending is None else ctx.sink.pending + d_values
            d_values = None
        return (d_values, None, d_psw if ctx.needs_input_grad[2] else None,
                d_hyp if ctx.needs_input_grad[3] else None, None, None, None, None, None)


def _final_values_step(values, indices, psw, d_hyp, scale, lr, wd, clip, out):
    """The values step of an update whose result is only stored (the last
    chunk's: no loss differentiates through it): pkm_eb_bwd_sgd writing the
    new table straight into `out` (the values parameter, which must not share
    storage with `values`), without the scaled gradient. Returns the per-row
    sums of the scaled gradient's squares."""
    from ..embedding_bag import eb_backward_workspace_bytes

    with torch.no_grad():
        V = _aligned(values.detach())
        idx = indices.contiguous()
        w = psw.detach().contiguous()
        g = _aligned(d_hyp.detach().to(V.dtype))
        K, D = V.shape
        B, L = idx.shape
        sumsq = torch.empty(K, dtype=torch.float32, device=V.device)
        ws_bytes = eb_backward_workspace_bytes(K, D, B, L)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=V.device)
        _lib.call("pkm_eb_bwd_sgd", _lib.ptr(V), K, D, _lib.dtype_code(V), _lib.ptr(idx), _lib.ptr(w),
                  _lib.dtype_code(w), _lib.ptr(g), B, L, float(scale), float(lr), float(wd), int(bool(clip)),
                  _lib.ptr(out), None, None, None, _lib.ptr(sumsq), _lib.ptr(ws), ws_bytes,
                  _lib.stream_of(V.device))
    return sumsq


def _storable_into(values: torch.Tensor, param: torch.Tensor) -> bool:
    """Whether the last values step can write the parameter directly: same
    shape and dtype, a 16-byte aligned contiguous parameter, no shared storage
    with the table the step reads."""
    if param.shape != values.shape or param.dtype != values.dtype or not param.is_contiguous():
        return False
    if param.data_ptr() % 16 or param.device != values.device:
        return False
    a0, a1 = param.data_ptr(), param.data_ptr() + param.numel() * param.element_size()
    b0 = values.untyped_storage().data_ptr()
    b1 = b0 + values.untyped_storage().nbytes()
    return a1 <= b0 or b1 <= a0


def sgd_value_update(p: torch.Tensor, g: torch.Tensor, indices: torch.Tensor, scale: float, lr: float,
                     weight_decay: float, grad_clip: bool):
    """The values branch of update_fw with the "sgd" optimizer
    (fwpkm.py:334-365, 266-272): returns (p - lr * (clip(g') + wd * p), g')
    with g' = g * scale / max(bincount(indices), 1) per row, both in p's
    dtype. float32 / bfloat16 / float16 tables on the GPU."""
    _require_device(p, g, indices)
    if p.dim() != 2 or p.shape != g.shape:
        raise ValueError(f"values and gradient must be the same [size, v_dim], got {tuple(p.shape)}, {tuple(g.shape)}")
    if p.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"values dtype {p.dtype} not supported (float32, bfloat16, float16 are)")
    counts = torch.bincount(indices.reshape(-1), minlength=p.shape[0])
    return _SgdValueUpdate.apply(p, g, counts, scale, lr, weight_decay, grad_clip)


def _chunks(T: int, first: int, size: int):
    """[(start, end)]: the first chunk ends at min(first, T), the rest are
    `size` long (the last one shorter)."""
    first = min(first, T)
    bounds = [(0, first)]
    bounds += [(s, min(s + size, T)) for s in range(first, T, size)]
    return bounds


def _sl(t: Optional[torch.Tensor], a: int, b: int) -> Optional[torch.Tensor]:
    return t[:, a:b].contiguous() if t is not None else None


class FastWeightProductKeyMemory(nn.Module):
    """Fast-weight product-key memory (fwpkm/fwpkm.py:22-934): product-key
    retrieval over `keys` / `values` that are updated in context, chunk by
    chunk, by one SGD step on a memorisation loss (and an addressing loss on
    the keys); the outer loss differentiates through those steps."""

    def __init__(
        self,
        mem_k_dim=512,
        mem_v_dim=512,
        mem_heads=1,
        mem_topk=8,
        mem_n_subkeys=512,
        lookahead=1,
        qk_score_type="idw",
        score_nonlinear="softmax",
        score_temperature=1.0,
        optimizer_type="sgd",
        learning_rate=1.0,
        weight_decay=0.0,
        loss_type="mse",
        mem_grad_to_values_only=True,
        grad_clip=False,
        addr_loss="me",
        addr_loss_weight=1.0,
        fp32_fw=True,
    ):
        assert mem_k_dim >= 2
        assert mem_k_dim % 2 == 0
        check_supported(mem_n_subkeys, mem_k_dim, mem_topk, mem_v_dim, "FastWeightProductKeyMemory")
        super().__init__()
        self.subsize = mem_n_subkeys
        self.size = mem_n_subkeys**2
        self.k_dim = mem_k_dim
        self.v_dim = mem_v_dim
        self.heads = mem_heads
        self.topk = mem_topk
        self.lookahead = lookahead
        self.qk_score_type = qk_score_type
        self.score_nonlinear = score_nonlinear
        self.score_temperature = score_temperature
        self.optimizer_type = optimizer_type
        self.learning_rate = learning_rate
        self.weight_decay = weight_decay
        self.loss_type = loss_type
        self.mem_grad_to_values_only = mem_grad_to_values_only
        self.grad_clip = grad_clip
        self.addr_loss = addr_loss
        self.addr_loss_weight = addr_loss_weight
        self.fp32_fw = fp32_fw
        # slot observation log (write_ob_log), off unless ob_mode is set
        self.ob_mode = None
        self.ob_idx2log = defaultdict(list)
        # key (h, c, i) is row (2h + c) * subsize + i; value slot i1 * subsize + i2
        self.keys = nn.Parameter(torch.zeros(2 * self.heads * self.subsize, self.k_dim // 2))
        self.values = nn.Parameter(torch.zeros(self.size, self.v_dim))

    def reset_parameters(self):
        """fwpkm.py:90-95: keys U(+-1/sqrt(k_dim)), values N(0, v_dim^-1/2)."""
        bound = 1 / math.sqrt(self.k_dim)
        nn.init.uniform_(self.keys, a=-bound, b=bound)
        nn.init.normal_(self.values, mean=0, std=self.v_dim**-0.5)

    def get_fw_named_params(self):
        """The fast weights an update chain starts from (float32 copies with
        fp32_fw; for float32 parameters, the parameters themselves)."""
        return OrderedDict((n, p.float() if self.fp32_fw else p) for n, p in self.named_parameters())

    # ---- retrieval ------------------------------------------------------------------------

    def compute_qk_scores(self, q, k):
        return compute_qk_scores(q, k, self.qk_score_type)

    def get_indices(self, query: torch.Tensor, keys: torch.Tensor):
        """(scores, indices, topk_indices1, topk_indices2 [BT, heads, topk],
        scores1, scores2 [BT, heads, subsize]) (fwpkm.py:871-934)."""
        return get_indices(query, keys, self.heads, self.k_dim, self.topk, self.qk_score_type)

    def score_transform(self, scores):
        """softmax / silu / relu of scores / temperature over the last dim
        (heads x topk jointly), in the scores' dtype (fwpkm.py:105-115)."""
        scores = scores / self.score_temperature
        if self.score_nonlinear == "softmax":
            return score_softmax(scores)
        if self.score_nonlinear == "silu":
            return F.silu(scores).type_as(scores)
        if self.score_nonlinear == "relu":
            return F.relu(scores).type_as(scores)
        raise NotImplementedError(f"Non-linear {self.score_nonlinear} not implemented for scores.")

    def retrieve_values(self, query: torch.Tensor, fw_named_params: OrderedDict):
        """query [B, T, heads * k_dim] -> dict of the retrieved values
        [B * T, v_dim] (key "retireved_values", spelled as the reference
        spells it), the top-k scores, their transform, the indices, the
        per-half indices and the full sub-score matrices (fwpkm.py:149-198)."""
        B, T = query.shape[:2]
        scores, indices, i1, i2, s1, s2 = self.get_indices(query.view(B * T, self.heads, self.k_dim),
                                                           fw_named_params["keys"])
        normed = self.score_transform(scores.view(B * T, self.heads * self.topk))
        vals = xformers_embedding_bag(indices=indices.view(B * T, self.heads * self.topk),
                                      weight=fw_named_params["values"], per_sample_weights=normed)
        return {
            "retireved_values": vals,
            "scores": scores,
            "normed_scores": normed,
            "indices": indices,
            "sub_indices1": i1,
            "sub_indices2": i2,
            "all_sub_scores1": s1,
            "all_sub_scores2": s2,
        }

    # ---- losses -----------------------------------------------------------------------------

    def compute_marginal_entropy(self, M, epsilon=1e-8):
        """Entropy of the batch-mean softmax over each row's top-k logits of M
        [N, K] (the rest masked to -inf) (fwpkm.py:117-147)."""
        if self.addr_loss_weight == 0.0:
            return torch.tensor(0.0, device=M.device, dtype=M.dtype)
        return self._marginal_entropy(M, torch.topk(M, self.topk, dim=1)[0][:, -1:], epsilon)

    @staticmethod
    def _marginal_entropy(M, kth, epsilon=1e-8):
        """compute_marginal_entropy with each row's k-th largest value kth [N, 1]
        given (it only enters the comparison, so it carries no gradient)."""
        masked = torch.where(M >= kth, M, torch.full_like(M, float("-inf")))
        p_bar = F.softmax(masked.float(), dim=1).mean(dim=0)
        return (-(p_bar * torch.log(p_bar + epsilon)).sum()).to(M.dtype)

    def compute_mem_loss(self, hyp_values, ref_values, loss_mask=None, loss_weights=None):
        """Per-example mean squared error [BT], times the optional mask and
        weights (fwpkm.py:200-231)."""
        if self.loss_type != "mse":
            raise NotImplementedError(f"Loss type {self.loss_type} not implemented.")
        losses = F.mse_loss(hyp_values, ref_values, reduction="none").mean(dim=-1)
        if loss_mask is not None:
            losses = losses * loss_mask
        if loss_weights is not None:
            losses = losses * loss_weights
        return losses

    def compute_addr_loss(self, sub_indices1, sub_indices2, all_sub_scores1, all_sub_scores2):
        """-(marginal entropy of each half's addressing), weighted, or None
        (fwpkm.py:233-264)."""
        if self.addr_loss is None:
            return None
        if self.addr_loss != "me":
            raise NotImplementedError(f"Addressing loss {self.addr_loss} not implemented.")
        if self.addr_loss_weight == 0.0:
            h1 = self.compute_marginal_entropy(all_sub_scores1.view(-1, self.subsize))
            h2 = self.compute_marginal_entropy(all_sub_scores2.view(-1, self.subsize))
            return self.addr_loss_weight * (-1.0 * h1 + -1.0 * h2)

        # each row's topk-th largest sub-score is that of its topk-th best sub-key
        # (the retrieval's per-half lists, best first): the value torch.topk gives
        def h(all_sub_scores, sub_indices):
            M = all_sub_scores.view(-1, self.subsize)
            kth = M.detach().gather(1, sub_indices.reshape(-1, self.topk)[:, -1:])
            return self._marginal_entropy(M, kth)

        return self.addr_loss_weight * (-1.0 * h(all_sub_scores1, sub_indices1) + -1.0 * h(all_sub_scores2, sub_indices2))

    # ---- inner update -----------------------------------------------------------------------

    def update_fw_param(self, p, g, lr, wd):
        if self.optimizer_type != "sgd":
            raise NotImplementedError(f"Optimizer {self.optimizer_type} not implemented.")
        return p - lr * (g + wd * p)

    def update_fw(self, fw_named_params: OrderedDict, num_samples: int, indices: torch.Tensor,
                  mem_loss: torch.Tensor, addr_loss: Optional[torch.Tensor] = None):
        """One SGD step of the fast weights on 0.5 * mem_loss (+ addr_loss)
        (fwpkm.py:274-367). Returns (updated params, unclipped gradients with
        the values' one scaled). The values' step runs as one kernel pass
        (sgd_value_update); create_graph follows self.training."""
        return self._update_fw(fw_named_params, num_samples, indices, mem_loss, addr_loss)

    def _update_fw(self, fw_named_params: OrderedDict, num_samples: int, indices: torch.Tensor,
                   mem_loss: torch.Tensor, addr_loss: Optional[torch.Tensor] = None, addr_grads=None):
        """update_fw; addr_grads: the address loss's gradient of each param,
        when the caller has it already (the marginal-entropy kernels): with
        mem_grad_to_values_only it replaces the autograd pass over addr_loss."""
        mem_loss = mem_loss * 0.5
        names = list(fw_named_params.keys())
        params = list(fw_named_params.values())
        if self.mem_grad_to_values_only:
            if addr_grads is not None:
                pass
            elif addr_loss is not None:
                addr_grads = torch.autograd.grad(addr_loss, params, create_graph=self.training, allow_unused=True)
            else:
                addr_grads = [None] * len(params)
            (g_values,) = torch.autograd.grad(mem_loss, fw_named_params["values"], create_graph=self.training)
            grads = [g_values if n == "values" else addr_grads[i] for i, n in enumerate(names)]
        else:
            loss = mem_loss if addr_loss is None else mem_loss + addr_loss
            grads = list(torch.autograd.grad(loss, params, create_graph=self.training))
        scale = num_samples * self.v_dim * self.topk * self.heads
        fused = self.optimizer_type == "sgd"
        scaled, updated = [], []
        for n, p, g in zip(names, params, grads):
            if n == "values" and fused and g is not None:
                new_p, g_scaled = sgd_value_update(p, g, indices, scale, self.learning_rate, self.weight_decay,
                                                   self.grad_clip)
                scaled.append(g_scaled)
                updated.append(new_p)
                continue
            if n == "values":
                counts = torch.bincount(indices.view(-1), minlength=self.size).to(g.dtype)
                counts[counts == 0] = 1.0
                g = (g * scale) / counts.unsqueeze(-1)
            scaled.append(g)
            step = torch.clamp(g, min=-1.0, max=1.0) if self.grad_clip else g
            updated.append(self.update_fw_param(p, step, self.learning_rate, self.weight_decay))
        return OrderedDict(zip(names, updated)), scaled

    def _fused_values_step(self, values: torch.Tensor) -> bool:
        """Whether the values step can run fused into the value backward
        (_FusedValueStep): the "sgd" optimizer, the memory loss's gradient to
        the values only, a float32 / bfloat16 table whose rows the backward's
        row kernels take whole (v_dim / (16 bytes / element) = 2^a * b, a <= 6,
        b in 1, 2, 4, 8)."""
        if self.optimizer_type != "sgd" or not self.mem_grad_to_values_only:
            return False
        if values.dtype not in (torch.float32, torch.bfloat16):
            return False
        nvec, epv = values.shape[1], 4 if values.dtype == torch.float32 else 8
        if nvec % epv:
            return False
        nvec //= epv
        return nvec <= 64 and (nvec & (nvec - 1)) == 0 or (nvec % 64 == 0 and nvec // 64 in (1, 2, 4, 8))

    def _update_fw_fused(self, fw_named_params: OrderedDict, num_samples: int, retrieval: dict,
                         mem_loss: torch.Tensor, addr_loss: Optional[torch.Tensor] = None,
                         store_into: Optional[torch.Tensor] = None, addr_grads=None):
        """update_fw with the values step fused into the value backward: the
        same step (fwpkm.py:333-365) and outer gradients, the table gradient
        and the dense normalisation / SGD passes replaced by one kernel.
        Returns (updated params, [scaled gradient of each param], [squared
        norm of each]: the values' from the kernel's row sums; the values'
        scaled gradient itself is None, its norm being all the caller reads).

        store_into: the values parameter, for the last chunk's step, whose
        result is only stored (fwpkm.py:540-545) and never differentiated: the
        new table is written into it directly, with no graph and no scaled
        gradient (its entry in the returned gradients is None).

        addr_grads: as in update_fw."""
        mem_loss = mem_loss * 0.5
        names = list(fw_named_params.keys())
        params = list(fw_named_params.values())
        if addr_grads is not None:
            pass
        elif addr_loss is not None:
            addr_grads = torch.autograd.grad(addr_loss, params, create_graph=self.training, allow_unused=True)
        else:
            addr_grads = [None] * len(params)
        hyp = retrieval["retireved_values"]
        if store_into is None:
            (d_hyp,) = torch.autograd.grad(mem_loss, hyp, create_graph=self.training)
        else:
            (d_hyp,) = torch.autograd.grad(mem_loss, hyp, retain_graph=True)
        scale = num_samples * self.v_dim * self.topk * self.heads
        flat = retrieval["indices"].reshape(hyp.shape[0], -1)
        psw = retrieval["normed_scores"].reshape(hyp.shape[0], -1)
        scaled, updated, norms2 = [], [], []
        for i, (n, p) in enumerate(zip(names, params)):
            if n == "values" and store_into is not None:
                sumsq = _final_values_step(p, flat, psw, d_hyp, scale, self.learning_rate, self.weight_decay,
                                           self.grad_clip, store_into)
                scaled.append(None)
                updated.append(store_into)
                norms2.append(sumsq.sum())
                continue
            if n == "values":
                # the scaled gradient is not needed here: its norm comes from the row sums
                new_p, g_scaled, sumsq = _FusedValueStep.apply(p, flat, psw, d_hyp, scale, self.learning_rate,
                                                               self.weight_decay, self.grad_clip, False)
                scaled.append(g_scaled)
                updated.append(new_p)
                norms2.append(sumsq.sum())
                continue
            g = addr_grads[i]
            scaled.append(g)
            step = torch.clamp(g, min=-1.0, max=1.0) if self.grad_clip else g
            updated.append(self.update_fw_param(p, step, self.learning_rate, self.weight_decay))
            norms2.append(None)
        return OrderedDict(zip(names, updated)), scaled, norms2

    def write_ob_log(self, token_ids, indices, scores):
        """Appends, per slot read, (query token, value token, up to 10 tokens
        of context either side of the value token, score) to ob_idx2log
        (fwpkm.py:369-393). token_ids [B, T]; indices, scores [B, T, heads * topk]."""
        assert self.ob_mode
        B, T = token_ids.shape
        ids = token_ids.tolist()
        la = self.lookahead
        for b in range(B):
            for t in range(T - la):
                v = t + la
                entry_ctx = (ids[b][t], ids[b][v], ids[b][max(0, v - 10):v], ids[b][v + 1:min(T, v + 10)])
                for j in range(self.heads * self.topk):
                    self.ob_idx2log[indices[b, t, j].item()].append(entry_ctx + (scores[b, t, j].item(),))

    def _update_targets(self, hyp, ref, gates, mask):
        """The (hyp, ref, weights, mask) the update fits: the last `lookahead`
        hypotheses (and their weights / mask) drop out, the targets shift by
        `lookahead` (fwpkm.py:464-486, 684-701)."""
        la = self.lookahead
        stop = None if la == 0 else -la
        return (hyp[:, :stop].contiguous(), ref[:, la:].contiguous(),
                gates[:, :stop].contiguous() if gates is not None else None,
                mask[:, :stop].contiguous() if mask is not None else None)

    def _losses(self, hyp, ref, weights, mask, retrieval, query=None, params=None, create_graph=False):
        """(per-example memory losses, address loss, the address loss's
        gradient of each param or None). The gradient comes with the loss from
        the marginal-entropy kernels when they apply (query and params given:
        the retrieval's query and the params it read); otherwise the caller
        differentiates the loss."""
        D = hyp.size(-1)
        mem_losses = self.compute_mem_loss(
            hyp_values=hyp.view(-1, D),
            ref_values=ref.view(-1, ref.size(-1)),
            loss_mask=mask.view(-1) if mask is not None else None,
            loss_weights=weights.view(-1) if weights is not None else None,
        )
        if self._addr_kernels(retrieval, query, params):
            addr_loss, g_keys = addr_loss_and_key_grad(
                query, params["keys"], retrieval["all_sub_scores1"], retrieval["all_sub_scores2"],
                retrieval["sub_indices1"], retrieval["sub_indices2"], self.heads, self.topk, self.addr_loss_weight,
                _score_type(self.qk_score_type), create_graph)
            return mem_losses, addr_loss, [g_keys if n == "keys" else None for n in params]
        addr_loss = self.compute_addr_loss(retrieval["sub_indices1"], retrieval["sub_indices2"],
                                           retrieval["all_sub_scores1"], retrieval["all_sub_scores2"])
        return mem_losses, addr_loss, None

    def _addr_kernels(self, retrieval, query, params) -> bool:
        """Whether the address loss and its gradient run on the
        marginal-entropy kernels: the "me" loss with a nonzero weight, the
        keys' gradient from it alone (mem_grad_to_values_only), one dtype for
        the query, keys and sub-scores, sizes the kernels take."""
        if query is None or params is None or "keys" not in params:
            return False
        if self.addr_loss != "me" or self.addr_loss_weight == 0.0 or not self.mem_grad_to_values_only:
            return False
        s1 = retrieval["all_sub_scores1"]
        keys = params["keys"]
        return (s1.dtype == keys.dtype == query.dtype
                and _me_supported(self.subsize, s1.dtype, _score_type(self.qk_score_type)))

    def _store_fast_weights(self, fw_named_params):
        with torch.no_grad():
            for n, p in self.named_parameters():
                if n in fw_named_params and fw_named_params[n] is not p:  # (the last step may have written p)
                    p.data.copy_(fw_named_params[n].data.to(p.dtype))

    # ---- chunked forward --------------------------------------------------------------------

    def forward_wo_past(self, q, ref_v, chunk_size, gates=None, loss_mask=None, token_ids=None):
        """Training / prefill: split T into chunks; each chunk reads the
        memory, then fits it with one update step whose result the next chunk
        reads; the outer graph runs through every step (fwpkm.py:395-558)."""
        B, T = q.shape[:2]
        input_dtype = q.dtype
        if self.fp32_fw:
            q, ref_v = q.float(), ref_v.float()
        outputs, indices, scores, losses, addr_losses, step_norms = [], [], [], [], [], []
        with torch.enable_grad():
            params = self.get_fw_named_params()
            n_params = len(params)
            fused = self._fused_values_step(params["values"])
            bounds = _chunks(T, chunk_size, chunk_size)
            # one split per tensor (its backward is one concatenation, not a zero-filled full-size
            # gradient per chunk added up)
            sizes = [e - s for s, e in bounds]
            q_chunks, ref_chunks = q.split(sizes, dim=1), ref_v.split(sizes, dim=1)
            for ci, (start, end) in enumerate(bounds):
                cT = end - start
                cgates, cmask, cids = _sl(gates, start, end), _sl(loss_mask, start, end), _sl(token_ids, start, end)
                cq = q_chunks[ci].contiguous()
                final = ci == len(bounds) - 1
                read_params = step_params = params
                if fused and not final and params["values"].requires_grad:
                    # the table's retrieval and update step meet in one gradient buffer
                    v_read, v_step = _fan_out(params["values"])
                    read_params = OrderedDict((n, v_read if n == "values" else p) for n, p in params.items())
                    step_params = OrderedDict((n, v_step if n == "values" else p) for n, p in params.items())
                r = self.retrieve_values(cq, read_params)
                hyp = r["retireved_values"].view(B, cT, -1)
                # the chunk's output is read before its own update
                outputs.append(hyp)
                indices.append(r["indices"].view(B, cT, -1))
                scores.append(r["normed_scores"].view(B, cT, -1))
                u_hyp, u_ref, u_w, u_mask = self._update_targets(hyp, ref_chunks[ci].contiguous(), cgates, cmask)
                # the last step's result is only stored, never differentiated
                mem_losses, addr_loss, addr_grads = self._losses(u_hyp, u_ref, u_w, u_mask, r, query=cq,
                                                                 params=params,
                                                                 create_graph=self.training and not final)
                num_samples = (u_mask > 0).sum().item() if u_mask is not None else B * cT
                if fused:
                    # the last step's table is written into the parameter when it can be
                    last = final and _storable_into(params["values"], self.values)
                    params, grads, norms2 = self._update_fw_fused(step_params, num_samples, r, mem_losses.mean(),
                                                                  addr_loss, self.values if last else None,
                                                                  addr_grads=addr_grads)
                else:
                    params, grads = self._update_fw(params, num_samples, r["indices"], mem_losses.mean(), addr_loss,
                                                    addr_grads=addr_grads)
                    norms2 = [None] * len(grads)
                if self.ob_mode:
                    self.write_ob_log(token_ids=cids.view(B, cT), indices=r["indices"].view(B, cT, -1),
                                      scores=cgates.view(B, cT, -1))
                with torch.no_grad():
                    # each param's gradient norm (the values' from the kernel's row sums when fused)
                    step_norms.append([torch.sqrt(n2).to(p.dtype) if n2 is not None else g.detach().norm()
                                       for g, n2, p in zip(grads, norms2, params.values())])
                losses.append(mem_losses.view(B, -1).detach())
                if self.addr_loss is not None:
                    addr_losses.append(addr_loss.detach())
        with torch.no_grad():
            grad_norms = [torch.stack([nr[i] for nr in step_norms]).mean() for i in range(n_params)]
        self._store_fast_weights(params)
        return {
            "output": torch.cat(outputs, dim=1).to(input_dtype),
            "indices": torch.cat(indices, dim=1).view(B, T, self.heads, self.topk),
            "scores": torch.cat(scores, dim=1).view(B, T, self.heads, self.topk),
            "losses": torch.cat(losses, dim=1),
            "addr_loss": torch.stack(addr_losses).mean() if self.addr_loss is not None else None,
            "grad_norms": grad_norms,
            "past_key_values": None,
        }

    def forward_w_past(self, q, ref_v, gates, chunk_size, loss_mask=None, past_key_values=None, token_ids=None):
        """Streaming (generation): tokens queue up with the unprocessed tail
        of earlier calls (past_key_values = (q, hyp_v, ref_v, gates, mask,
        ids) queues); the memory is fitted on a queue once it holds a chunk
        (fwpkm.py:560-820)."""
        B, T = q.shape[:2]
        input_dtype = q.dtype
        if self.fp32_fw:
            q, ref_v = q.float(), ref_v.float()
        dev, dt = ref_v.device, ref_v.dtype

        def empty(width=None, dtype=dt):
            return torch.zeros((B, 0) if width is None else (B, 0, width), device=dev, dtype=dtype)

        qq, hq, rq = empty(q.size(-1)), empty(ref_v.size(-1)), empty(ref_v.size(-1))
        gq = empty() if gates is not None else None
        mq = empty() if loss_mask is not None else None
        iq = empty(dtype=torch.long) if token_ids is not None else None
        if past_key_values is not None:
            p_q, p_h, p_r, p_g, p_m, p_i = past_key_values
            if p_h is not None:
                assert p_h.size(1) < chunk_size + self.lookahead, (
                    f"Past key values length {p_h.size(1)} longer than "
                    f"chunk size + lookahead ({chunk_size} + {self.lookahead})."
                )
                qq, hq, rq = torch.cat([p_q, qq], 1), torch.cat([p_h, hq], 1), torch.cat([p_r, rq], 1)
                gq = torch.cat([p_g, gq], 1) if gates is not None else None
                mq = torch.cat([p_m, mq], 1) if loss_mask is not None else None
                iq = torch.cat([p_i, iq], 1) if token_ids is not None else None

        la = self.lookahead
        stop = None if la == 0 else -la
        updated = False
        params = self.get_fw_named_params()
        outputs, indices, scores, losses, addr_losses = [], [], [], [], []
        for start, end in _chunks(T, chunk_size + la - rq.size(1), chunk_size):
            cT = end - start
            cq = q[:, start:end, :].contiguous()
            cgates, cmask, cids = _sl(gates, start, end), _sl(loss_mask, start, end), _sl(token_ids, start, end)
            r = self.retrieve_values(cq, params)
            hyp = r["retireved_values"].view(B, cT, -1)
            chunk_indices = r["indices"]
            outputs.append(hyp)
            indices.append(chunk_indices.view(B, cT, -1))
            scores.append(r["normed_scores"].view(B, cT, -1))
            qq, hq, rq = torch.cat([qq, cq], 1), torch.cat([hq, hyp], 1), torch.cat([rq, ref_v[:, start:end]], 1)
            gq = torch.cat([gq, cgates], 1) if gates is not None else None
            mq = torch.cat([mq, cmask], 1) if loss_mask is not None else None
            iq = torch.cat([iq, cids], 1) if token_ids is not None else None
            if past_key_values and hq.size(1) < chunk_size:
                continue  # not a chunk's worth of signal yet
            updated = True
            with torch.enable_grad():
                params = {n: p.detach().requires_grad_(True) for n, p in params.items()}
                uq = qq[:, :stop].contiguous()
                ru = self.retrieve_values(uq, params)
                u_w = gq[:, :stop].contiguous() if gq is not None else None
                u_mask = mq[:, :stop].contiguous() if mq is not None else None
                mem_losses, addr_loss, addr_grads = self._losses(ru["retireved_values"], rq[:, la:].contiguous(),
                                                                 u_w, u_mask, ru, query=uq, params=params,
                                                                 create_graph=self.training)
                # as the reference: samples counted as B * chunk length, slots from the forward chunk
                num_samples = (u_mask > 0).sum().item() if u_mask is not None else B * cT
                params, _ = self._update_fw(params, num_samples, chunk_indices, mem_losses.mean(), addr_loss,
                                            addr_grads=addr_grads)
                if self.ob_mode:
                    pad = torch.zeros(iq.size(0), la, self.heads * self.topk, device=iq.device)
                    n_u = iq.size(1) - la
                    self.write_ob_log(
                        token_ids=iq,
                        indices=torch.cat([ru["indices"].view(B, n_u, -1), pad.to(ru["indices"].dtype)], 1),
                        scores=torch.cat([ru["scores"].view(B, n_u, -1), pad.to(ru["scores"].dtype)], 1),
                    )
            if la == 0:
                qq, hq, rq = empty(q.size(-1)), empty(ref_v.size(-1)), empty(ref_v.size(-1))
                gq = empty() if gates is not None else None
                mq = empty() if loss_mask is not None else None
                iq = empty(dtype=torch.long)
            else:
                qq, hq, rq = qq[:, -la:].contiguous(), hq[:, -la:].contiguous(), rq[:, -la:].contiguous()
                gq = gq[:, -la:].contiguous() if gates is not None else None
                mq = mq[:, -la:].contiguous() if u_mask is not None else None
                # (the reference slices the id queue unconditionally and fails without token ids)
                iq = iq[:, -la:].contiguous() if iq is not None else None
            losses.append(mem_losses.view(B, -1).detach())
            if self.addr_loss is not None:
                addr_losses.append(addr_loss.detach())
        if updated:
            self._store_fast_weights(params)
        return {
            "output": torch.cat(outputs, dim=1).to(input_dtype),
            "indices": torch.cat(indices, dim=1).view(B, T, self.heads, self.topk),
            "scores": torch.cat(scores, dim=1).view(B, T, self.heads, self.topk),
            "losses": torch.cat(losses, dim=1) if updated else None,
            "addr_loss": torch.stack(addr_losses).mean() if (updated and self.addr_loss is not None) else None,
            "grad_norms": None,
            "past_key_values": (qq, hq, rq, gq, mq, iq),
        }

    @torch.compiler.disable(recursive=True)
    def forward(self, q, ref_v, gates, chunk_size, loss_mask=None, past_key_values=None, token_ids=None):
        """Dict of output [B, T, v_dim], indices / scores [B, T, heads, topk],
        losses, addr_loss, grad_norms, past_key_values (fwpkm.py:822-851)."""
        if past_key_values is None:
            return self.forward_wo_past(q=q, ref_v=ref_v, gates=gates, chunk_size=chunk_size, loss_mask=loss_mask,
                                        token_ids=token_ids)
        return self.forward_w_past(q=q, ref_v=ref_v, gates=gates, chunk_size=chunk_size, loss_mask=loss_mask,
                                   past_key_values=past_key_values, token_ids=token_ids)


__all__ = ["FastWeightProductKeyMemory", "l2norm", "get_indices", "compute_qk_scores", "sgd_value_update"]
