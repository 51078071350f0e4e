"""Fast-weight PKM (FwPKM) chunk loop: CPU restatement (test infrastructure only).

A functional restatement of FastWeightProductKeyMemory (fwpkm/fwpkm.py) over
explicit tensors, differentiable end to end with torch autograd (create_graph
through the inner step), in any dtype:

  retrieve (fwpkm.py:149-198, 853-934):
    s_c  = score(q_c, K_c)                  dot, or idw -log(1e-3 + cdist(q, k)^2)
    sel  = per-half top-k, cartesian top-k  (oracle.pkm.select; or a given selection)
    sc   = s_0[i_0] + s_1[i_1]              [BT, H, k] in the dtype
    w    = transform(sc / temperature)      softmax / silu / relu over H * k jointly (:105-115)
    hyp  = sum_j w_j V[idx_j]               index_select + sum (grad_wrapper:98-103); the
                                            backward reads the saved table (grad_wrapper:119-155)
  per chunk of forward_wo_past (fwpkm.py:395-558):
    hyp is read before the chunk's update; lookahead shifts targets (:464-486)
    L_mem = mean over examples of mse(hyp, ref).mean(-1) * mask * gates (:200-231)
    L_addr = -w_a (H(P_0) + H(P_1)), H the entropy of the batch-mean softmax
             over each row's top-k sub-scores (:117-147, 233-264)
    grads  = d(0.5 L_mem)/dV (+ d L_addr / d keys), create_graph (:296-331)
    V'     = V - lr (clip(g * scale / max(count, 1)) + wd V),
             scale = samples * v_dim * k * H (:333-365); keys likewise unscaled
  forward_w_past (fwpkm.py:560-820): queues of (q, hyp, ref, gates, mask, ids)
    across calls; an update fits the queue once it holds a chunk.
  After the loop the module stores the last fast weights into its parameters
  in place (fwpkm.py:540-545). Where the chain starts from the parameters
  themselves (float32 parameters with fp32_fw, or fp32_fw off), the first
  chunk's graph saved those tensors, so its outer backward reads the stored
  (updated) table and keys: the reference's gradients include that, and so
  do this restatement's (keys / values passed in are updated in place).

Pinned by tests/test_oracle_fwpkm.py against the reference's own outputs
(tests/golden/fwpkm_*.pt, written by importing fwpkm/fwpkm.py on the CPU).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import torch
import torch.nn.functional as F

from . import pkm as pkm_ref


@dataclass
class FwConfig:
    heads: int
    k_dim: int
    v_dim: int
    topk: int
    subsize: int
    lookahead: int = 1
    score_type: str = "idw"  # "dot_product" | "idw"
    score_nonlinear: str = "softmax"
    score_temperature: float = 1.0
    learning_rate: float = 1.0
    weight_decay: float = 0.0
    grad_clip: bool = False
    addr_loss: Optional[str] = "me"
    addr_loss_weight: float = 1.0
    mem_grad_to_values_only: bool = True
    fp32_fw: bool = True

    @staticmethod
    def from_module_kwargs(kw: dict) -> "FwConfig":
        return FwConfig(
            heads=kw.get("mem_heads", 1), k_dim=kw.get("mem_k_dim", 512), v_dim=kw.get("mem_v_dim", 512),
            topk=kw.get("mem_topk", 8), subsize=kw.get("mem_n_subkeys", 512), lookahead=kw.get("lookahead", 1),
            score_type=kw.get("qk_score_type", "idw"), score_nonlinear=kw.get("score_nonlinear", "softmax"),
            score_temperature=kw.get("score_temperature", 1.0), learning_rate=kw.get("learning_rate", 1.0),
            weight_decay=kw.get("weight_decay", 0.0), grad_clip=kw.get("grad_clip", False),
            addr_loss=kw.get("addr_loss", "me"), addr_loss_weight=kw.get("addr_loss_weight", 1.0),
            mem_grad_to_values_only=kw.get("mem_grad_to_values_only", True), fp32_fw=kw.get("fp32_fw", True))


def sub_scores(q: torch.Tensor, keys: torch.Tensor, cfg: FwConfig):
    """Differentiable s_0, s_1 [BT, H, n] in q's dtype (fwpkm.py:853-869, 891-905)."""
    BT = q.shape[0]
    half = cfg.k_dim // 2
    q = q.reshape(BT, cfg.heads, cfg.k_dim)
    K = keys.reshape(cfg.heads, 2, -1, half)
    out = []
    for c in range(2):
        qc, Kc = q[:, :, c * half:(c + 1) * half], K[:, c]
        if cfg.score_type == "dot_product":
            out.append(torch.einsum("bhd,hnd->bhn", qc, Kc))
        else:
            # the reference's own expression (fwpkm.py:863-866): its backward reads the distances
            # saved by the forward and the key table as it is when the backward runs
            dist = torch.cdist(qc.permute(1, 0, 2), Kc, p=2, compute_mode="use_mm_for_euclid_dist")
            out.append(-torch.log(1e-3 + dist.permute(1, 0, 2).pow(2)))
    return out[0], out[1]


def transform(scores: torch.Tensor, cfg: FwConfig) -> torch.Tensor:
    s = scores / cfg.score_temperature
    if cfg.score_nonlinear == "softmax":
        return F.softmax(s.float(), dim=-1).to(s.dtype)
    if cfg.score_nonlinear == "silu":
        return F.silu(s)
    if cfg.score_nonlinear == "relu":
        return F.relu(s)
    raise ValueError(cfg.score_nonlinear)


class _Bag(torch.autograd.Function):
    """sum_j w_j V[idx_j] with the reference's autograd structure
    (grad_wrapper:83-155): the table itself is saved and read again by the
    backward (index_select of the saved table), whose ops are recorded under
    create_graph, so the double backward is autograd's."""

    @staticmethod
    def forward(ctx, values, flat, w):
        ctx.save_for_backward(values, flat, w)
        acc = torch.float64 if values.dtype == torch.float64 else torch.float32
        return (values[flat].to(acc) * w.to(acc)[..., None]).sum(1).to(values.dtype)

    @staticmethod
    def backward(ctx, g):
        values, flat, w = ctx.saved_tensors
        acc = torch.float64 if values.dtype == torch.float64 else torch.float32
        contrib = (g.to(acc)[:, None, :] * w.to(acc)[..., None]).reshape(-1, values.shape[1])
        gW = torch.zeros(values.shape, dtype=acc).index_add(0, flat.reshape(-1), contrib).to(values.dtype)
        gw = (values[flat].to(acc) * g.to(acc)[:, None, :]).sum(-1).to(w.dtype)
        return gW, None, gw


def retrieve(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, cfg: FwConfig,
             idx: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
    """q [B, T, H * k_dim] -> retrieved values [B * T, v_dim] and the
    selection (fwpkm.py:149-198). `idx` [B * T, H, topk] forces the selection."""
    B, T = q.shape[:2]
    s1, s2 = sub_scores(q.reshape(B * T, cfg.heads, cfg.k_dim), keys, cfg)
    if idx is None:
        with torch.no_grad():
            _, idx, _, _ = pkm_ref.select(s1.detach(), s2.detach(), cfg.topk)
    idx = idx.reshape(B * T, cfg.heads, cfg.topk)
    n = cfg.subsize
    sc = s1.gather(2, idx // n) + s2.gather(2, idx % n)
    w = transform(sc.reshape(B * T, cfg.heads * cfg.topk), cfg)
    hyp = _Bag.apply(values, idx.reshape(B * T, cfg.heads * cfg.topk), w)
    # sum over the bag of |w| |V[idx]|: the scale of each retrieved value's terms (a test's
    # rounding bound for sums with cancellation), no gradient
    with torch.no_grad():
        mag = _Bag.apply(values.detach().abs(), idx.reshape(B * T, cfg.heads * cfg.topk), w.detach().abs())
    return {"hyp": hyp, "scores": sc, "normed": w, "indices": idx, "s1": s1, "s2": s2, "mag": mag}


def marginal_entropy(M: torch.Tensor, cfg: FwConfig, eps: float = 1e-8, M_sel: Optional[torch.Tensor] = None
                     ) -> torch.Tensor:
    """fwpkm.py:117-147. M_sel, when given, decides which entries are kept
    (>= the row's k-th largest of M_sel): another implementation's own
    (rounded) scores, so that ties at the threshold resolve as they did there."""
    if cfg.addr_loss_weight == 0.0:
        return torch.zeros((), dtype=M.dtype)
    S = M if M_sel is None else M_sel.to(M.device)
    kth = torch.topk(S, cfg.topk, dim=1)[0][:, -1:]
    P = F.softmax(torch.where(S >= kth, M, torch.full_like(M, float("-inf"))).float(), dim=1)
    p_bar = P.mean(0)
    return (-(p_bar * torch.log(p_bar + eps)).sum()).to(M.dtype)


def addr_loss(r, cfg: FwConfig, sel_scores=None):
    if cfg.addr_loss is None:
        return None
    m1, m2 = (None, None) if sel_scores is None else (t.reshape(-1, cfg.subsize) for t in sel_scores)
    h1 = marginal_entropy(r["s1"].reshape(-1, cfg.subsize), cfg, M_sel=m1)
    h2 = marginal_entropy(r["s2"].reshape(-1, cfg.subsize), cfg, M_sel=m2)
    return cfg.addr_loss_weight * (-h1 - h2)


def mem_losses(hyp, ref, mask, weights):
    out = ((hyp - ref) ** 2).mean(-1)
    if mask is not None:
        out = out * mask
    if weights is not None:
        out = out * weights
    return out


def update(params: Dict[str, torch.Tensor], cfg: FwConfig, num_samples: int, indices: torch.Tensor,
           mem_loss: torch.Tensor, a_loss: Optional[torch.Tensor]):
    """One SGD step (fwpkm.py:274-367, 266-272); returns (new params, scaled grads)."""
    names = list(params)
    mem_loss = mem_loss * 0.5
    if cfg.mem_grad_to_values_only:
        if a_loss is not None:
            ag = torch.autograd.grad(a_loss, [params[n] for n in names], create_graph=True, allow_unused=True)
        else:
            ag = [None] * len(names)
        (gv,) = torch.autograd.grad(mem_loss, params["values"], create_graph=True)
        grads = [gv if n == "values" else ag[i] for i, n in enumerate(names)]
    else:
        total = mem_loss if a_loss is None else mem_loss + a_loss
        grads = list(torch.autograd.grad(total, [params[n] for n in names], create_graph=True))
    new, scaled = {}, []
    for n, g in zip(names, grads):
        p = params[n]
        if n == "values":
            cnt = torch.bincount(indices.reshape(-1), minlength=p.shape[0]).to(g.dtype)
            cnt = torch.where(cnt == 0, torch.ones_like(cnt), cnt)
            g = g * (num_samples * cfg.v_dim * cfg.topk * cfg.heads) / cnt[:, None]
        scaled.append(g)
        step = g.clamp(-1.0, 1.0) if cfg.grad_clip else g
        new[n] = p - cfg.learning_rate * (step + cfg.weight_decay * p)
    return new, scaled


def _targets(hyp, ref, gates, mask, la):
    stop = None if la == 0 else -la
    return (hyp[:, :stop], ref[:, la:], gates[:, :stop] if gates is not None else None,
            mask[:, :stop] if mask is not None else None)


def forward_wo_past(q, ref_v, keys, values, cfg: FwConfig, chunk_size: int, gates=None, loss_mask=None,
                    selections: Optional[List[torch.Tensor]] = None, sel_scores: Optional[list] = None):
    """fwpkm.py:395-558 on explicit tensors (keys / values are the module's
    parameters: the outer gradient reaches them). `selections`, when given,
    forces each chunk's retrieval (in call order); `sel_scores` [(s1, s2)]
    decides the address loss's top-k masks (marginal_entropy)."""
    B, T = q.shape[:2]
    in_dtype = q.dtype
    v0_abs = values.detach().abs().to(torch.float64)
    if cfg.fp32_fw:
        q, ref_v = q.float(), ref_v.float()
        params = {"keys": keys.float(), "values": values.float()}
    else:
        params = {"keys": keys, "values": values}
    outs, idxs, scs, losses, alosses, steps, mags, step_mags = [], [], [], [], [], [], [], []
    sel_iter = iter(selections) if selections is not None else None
    score_iter = iter(sel_scores) if sel_scores is not None else None
    for s in range(0, T, chunk_size):
        e = min(s + chunk_size, T)
        cT = e - s
        r = retrieve(q[:, s:e], params["keys"], params["values"], cfg, next(sel_iter) if sel_iter else None)
        hyp = r["hyp"].reshape(B, cT, -1)
        outs.append(hyp)
        mags.append(r["mag"].reshape(B, cT, -1))
        idxs.append(r["indices"].reshape(B, cT, -1))
        scs.append(r["normed"].reshape(B, cT, -1))
        cg = gates[:, s:e] if gates is not None else None
        cm = loss_mask[:, s:e] if loss_mask is not None else None
        u_hyp, u_ref, u_w, u_m = _targets(hyp, ref_v[:, s:e], cg, cm, cfg.lookahead)
        ml = mem_losses(u_hyp.reshape(-1, u_hyp.shape[-1]), u_ref.reshape(-1, u_ref.shape[-1]),
                        u_m.reshape(-1) if u_m is not None else None, u_w.reshape(-1) if u_w is not None else None)
        al = addr_loss(r, cfg, next(score_iter) if score_iter else None)
        ns = int((u_m > 0).sum()) if u_m is not None else B * cT
        if cfg.mem_grad_to_values_only:
            # the scale of this chunk's value step: lr * scale / count * sum over the lookups of
            # |w| |dL/dhyp| (the terms of the value gradient's sums), no gradient
            (dh,) = torch.autograd.grad(0.5 * ml.mean(), r["hyp"], retain_graph=True)
            v = params["values"]
            with torch.no_grad():
                ix = r["indices"].reshape(-1)
                contrib = (r["normed"].detach().abs().reshape(-1, 1)
                           * dh.abs().repeat_interleave(cfg.heads * cfg.topk, 0))
                gabs = torch.zeros(v.shape, dtype=contrib.dtype).index_add_(0, ix, contrib)
                cnt = torch.bincount(ix, minlength=v.shape[0]).clamp_min(1).to(gabs.dtype)
                step_mags.append(cfg.learning_rate * gabs * (ns * cfg.v_dim * cfg.topk * cfg.heads) / cnt[:, None])
        params, g = update(params, cfg, ns, r["indices"], ml.mean(), al)
        steps.append([x.detach() for x in g])
        losses.append(ml.reshape(B, -1).detach())
        if al is not None:
            alosses.append(al.detach())
    # the module stores the last fast weights into its parameters in place
    # (fwpkm.py:540-545); where the chain started from the parameters
    # themselves, the first chunk's graph saved them, so the outer backward
    # of that chunk reads the stored (updated) values
    with torch.no_grad():
        keys.data.copy_(params["keys"].data.to(keys.dtype))
        values.data.copy_(params["values"].data.to(values.dtype))
    return {
        "output": torch.cat(outs, 1).to(in_dtype),
        "output_mag": torch.cat(mags, 1),
        # |initial values| + the chunks' value-step scales: the final values' rounding bound
        "values_mag": (v0_abs + sum(m.to(torch.float64) for m in step_mags)) if step_mags else None,
        "indices": torch.cat(idxs, 1).reshape(B, T, cfg.heads, cfg.topk),
        "scores": torch.cat(scs, 1).reshape(B, T, cfg.heads, cfg.topk),
        "losses": torch.cat(losses, 1),
        "addr_loss": torch.stack(alosses).mean() if alosses else None,
        "grad_norms": [torch.stack([st[i].norm() for st in steps]).mean() for i in range(2)],
        "final": {n: p.detach().to(keys.dtype if n == "keys" else values.dtype) for n, p in params.items()},
    }


def forward_w_past(q, ref_v, keys, values, cfg: FwConfig, chunk_size: int, gates=None, loss_mask=None,
                   past=None, token_ids=None):
    """fwpkm.py:560-820 on explicit tensors; returns the outputs, the queues
    and the fast weights after the call (None where no update happened)."""
    B, T = q.shape[:2]
    in_dtype = q.dtype
    if cfg.fp32_fw:
        q, ref_v = q.float(), ref_v.float()
    dt = ref_v.dtype
    z = lambda *shape, dtype=dt: torch.zeros((B, 0) + shape, dtype=dtype)  # noqa: E731
    qq, hq, rq = z(q.shape[-1]), z(ref_v.shape[-1]), z(ref_v.shape[-1])
    gq = z() if gates is not None else None
    mq = z() if loss_mask is not None else None
    iq = z(dtype=torch.long) if token_ids is not None else None
    if past is not None and past[1] is not None:
        qq, hq, rq = torch.cat([past[0], qq], 1), torch.cat([past[1], hq], 1), torch.cat([past[2], rq], 1)
        gq = torch.cat([past[3], gq], 1) if gates is not None else None
        mq = torch.cat([past[4], mq], 1) if loss_mask is not None else None
        iq = torch.cat([past[5], iq], 1) if token_ids is not None else None
    la = cfg.lookahead
    stop = None if la == 0 else -la
    params = {"keys": keys.float(), "values": values.float()} if cfg.fp32_fw else {"keys": keys, "values": values}
    first = min(chunk_size + la - rq.shape[1], T)
    bounds = [(0, first)] + [(s, min(s + chunk_size, T)) for s in range(first, T, chunk_size)]
    updated = False
    outs, idxs, scs, losses = [], [], [], []
    for s, e in bounds:
        cT = e - s
        r = retrieve(q[:, s:e], params["keys"], params["values"], cfg)
        hyp = r["hyp"].reshape(B, cT, -1)
        outs.append(hyp)
        idxs.append(r["indices"].reshape(B, cT, -1))
        scs.append(r["normed"].reshape(B, cT, -1))
        qq, hq, rq = torch.cat([qq, q[:, s:e]], 1), torch.cat([hq, hyp], 1), torch.cat([rq, ref_v[:, s:e]], 1)
        gq = torch.cat([gq, gates[:, s:e]], 1) if gates is not None else None
        mq = torch.cat([mq, loss_mask[:, s:e]], 1) if loss_mask is not None else None
        iq = torch.cat([iq, token_ids[:, s:e]], 1) if token_ids is not None else None
        if past is not None and hq.shape[1] < chunk_size:
            continue
        updated = True
        with torch.enable_grad():
            params = {n: p.detach().requires_grad_(True) for n, p in params.items()}
            ru = retrieve(qq[:, :stop], params["keys"], params["values"], cfg)
            u_w = gq[:, :stop] if gq is not None else None
            u_m = mq[:, :stop] if mq is not None else None
            ml = mem_losses(ru["hyp"], rq[:, la:].reshape(-1, rq.shape[-1]),
                            u_m.reshape(-1) if u_m is not None else None,
                            u_w.reshape(-1) if u_w is not None else None)
            ns = int((u_m > 0).sum()) if u_m is not None else B * cT
            params, _ = update(params, cfg, ns, r["indices"], ml.mean(), addr_loss(ru, cfg))
        if la == 0:
            qq, hq, rq = z(q.shape[-1]), z(ref_v.shape[-1]), z(ref_v.shape[-1])
            gq = z() if gates is not None else None
            mq = z() if loss_mask is not None else None
            iq = z(dtype=torch.long)
        else:
            qq, hq, rq = qq[:, -la:], hq[:, -la:], rq[:, -la:]
            gq = gq[:, -la:] if gates is not None else None
            mq = mq[:, -la:] if loss_mask is not None else None
            iq = iq[:, -la:] if iq is not None else None
        losses.append(ml.reshape(B, -1).detach())
    return {
        "output": torch.cat(outs, 1).to(in_dtype),
        "indices": torch.cat(idxs, 1).reshape(B, T, cfg.heads, cfg.topk),
        "scores": torch.cat(scs, 1).reshape(B, T, cfg.heads, cfg.topk),
        "losses": torch.cat(losses, 1) if updated else None,
        "queues": (qq, hq, rq, gq, mq, iq),
        "final": ({n: p.detach().to(keys.dtype if n == "keys" else values.dtype) for n, p in params.items()}
                  if updated else None),
    }
