"""Drop-in for the reference's fwpkm/fwmlp.py: the dense fast-weight MLP.

FastWeightMLP is the `fwpkm_variant="mlp"` alternative the modeling code can
build instead of the product-key memory (modeling_qwen3pkm.py:370-379): a
SwiGLU MLP (w_up / w_gate [size, input_dim], w_down [output_dim, size] and
biases) whose weights are fitted in context, chunk by chunk, by one SGD step
on a memorisation loss, with the outer graph running through every step
(fwmlp.py:20-522). It has no product-key lookup and no kernel of its own:
dense torch products on whatever device its tensors live on. Constructor,
parameter names, methods and return dicts are the reference's; so are its
quirks (the streaming path's update slices `[:-lookahead]`, which is empty
for lookahead 0, fwmlp.py:445-449).
"""
from __future__ import annotations

from collections import OrderedDict
from logging import getLogger
import math
from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from .fwpkm import l2norm  # noqa: F401  (the reference module defines it too, fwmlp.py:14-17)

logger = getLogger()


class FastWeightMLP(nn.Module):
    """Fast-weight SwiGLU MLP (fwmlp.py:20-522)."""

    def __init__(
        self,
        input_dim,
        output_dim,
        size,
        lookahead=0,
        lookahead_strategy="mean",
        optimizer_type="sgd",
        learning_rate=0.1,
        weight_decay=0.0,
        loss_type="mse",
        grad_clip=True,
        fp32_fw=True,
    ):
        super().__init__()
        self.input_dim = input_dim
        self.output_dim = output_dim
        self.size = size
        self.lookahead = lookahead
        self.lookahead_strategy = lookahead_strategy
        self.optimizer_type = optimizer_type
        self.learning_rate = learning_rate
        self.weight_decay = weight_decay
        self.loss_type = loss_type
        self.grad_clip = grad_clip
        self.fp32_fw = fp32_fw
        self.w_up = nn.Parameter(torch.ones(size, input_dim))
        self.b_up = nn.Parameter(torch.zeros(size))
        self.w_gate = nn.Parameter(torch.ones(size, input_dim))
        self.b_gate = nn.Parameter(torch.zeros(size))
        self.w_down = nn.Parameter(torch.ones(output_dim, size))
        self.b_down = nn.Parameter(torch.zeros(output_dim))

    def reset_parameters(self):
        """fwmlp.py:64-70: N(0, 1/sqrt(fan-in)) weights, zero biases."""
        for w, fan_in in ((self.w_up, self.input_dim), (self.w_gate, self.input_dim), (self.w_down, self.size)):
            nn.init.normal_(w, mean=0, std=1 / math.sqrt(fan_in))
        for b in (self.b_up, self.b_gate, self.b_down):
            nn.init.zeros_(b)

    def get_fw_named_params(self):
        return OrderedDict((n, p.float() if self.fp32_fw else p) for n, p in self.named_parameters())

    def update_fw_param(self, p, g, lr, wd):
        if self.optimizer_type != "sgd":
            raise NotImplementedError(f"Optimizer {self.optimizer_type} not implemented for fast weights.")
        return p - lr * (g + wd * p)

    def compute_mem_loss(self, hyp_values, ref_values, loss_mask: Optional[torch.Tensor] = None):
        """Per-example mean squared (or absolute) error [BT], times the mask (fwmlp.py:90-118)."""
        if self.loss_type == "mse":
            losses = F.mse_loss(hyp_values, ref_values, reduction="none").mean(dim=-1)
        elif self.loss_type == "mae":
            losses = (hyp_values - ref_values).abs().mean(dim=-1)
        else:
            raise NotImplementedError(f"Loss type {self.loss_type} not implemented.")
        return losses * loss_mask if loss_mask is not None else losses

    def retrieve_values(self, query, fw_named_params):
        """query [B, T, input_dim] -> {"retireved_values": [B * T, output_dim]}:
        w_down (up * silu(gate)) + b_down (fwmlp.py:120-149)."""
        B, T = query.shape[:2]
        x = query.view(B * T, self.input_dim)
        p = fw_named_params
        hidden = F.linear(x, p["w_up"], p["b_up"]) * F.silu(F.linear(x, p["w_gate"], p["b_gate"]))
        return {"retireved_values": F.linear(hidden, p["w_down"], p["b_down"])}

    def update_fw(self, fw_named_params, loss):
        """One SGD step of every fast weight on `loss` (fwmlp.py:151-186);
        returns (updated params, unclipped gradients)."""
        params = tuple(fw_named_params.values())
        grads = torch.autograd.grad(loss, params, create_graph=self.training)
        steps = [torch.clamp(g, min=-1.0, max=1.0) for g in grads] if self.grad_clip else grads
        new = [self.update_fw_param(p, g, self.learning_rate, self.weight_decay) for p, g in zip(params, steps)]
        return OrderedDict(zip(fw_named_params.keys(), new)), grads

    def _targets(self, ref):
        """Targets of the update: the mean of the lookahead + 1 shifted windows
        ("mean") or the last one ("last") (fwmlp.py:232-243)."""
        la = self.lookahead
        if la == 0:
            return ref
        windows = [ref[:, i:(i - la if i < la else None)] for i in range(la + 1)]
        if self.lookahead_strategy == "mean":
            return torch.stack(windows, dim=0).mean(dim=0)
        if self.lookahead_strategy == "last":
            return windows[-1]
        raise NotImplementedError(f"Lookahead strategy {self.lookahead_strategy} not implemented.")

    def forward_wo_past(self, q, ref_v, chunk_size, loss_mask=None):
        """Chunked in-context fitting over the whole sequence (fwmlp.py:188-297)."""
        B, T = q.shape[:2]
        input_dtype = q.dtype
        if self.fp32_fw:
            q, ref_v = q.float(), ref_v.float()
        la = self.lookahead
        stop = None if la == 0 else -la
        outputs, losses, step_grads = [], [], []
        with torch.enable_grad():
            params = self.get_fw_named_params()
            n_params = len(params)
            for start in range(0, T, chunk_size):
                end = min(start + chunk_size, T)
                cT = end - start
                hyp = self.retrieve_values(q[:, start:end].contiguous(), params)["retireved_values"].view(B, cT, -1)
                outputs.append(hyp)
                mask = loss_mask[:, start:end].contiguous()[:, :stop].contiguous() if loss_mask is not None else None
                u_hyp = hyp[:, :stop].contiguous()
                u_ref = self._targets(ref_v[:, start:end].contiguous()).contiguous()
                mem_losses = self.compute_mem_loss(u_hyp.view(-1, u_hyp.size(-1)), u_ref.view(-1, u_ref.size(-1)),
                                                   mask.view(-1) if mask is not None else None)
                params, grads = self.update_fw(params, mem_losses.mean())
                step_grads.append([g.detach() for g in grads])
                losses.append(mem_losses.view(B, -1).detach())
        with torch.no_grad():
            grad_norms = [torch.stack([g[i].norm() for g in step_grads]).mean() for i in range(n_params)]
            for n, p in self.named_parameters():
                if n in params:
                    p.data.copy_(params[n].data.to(p.dtype))
        return {
            "output": torch.cat(outputs, dim=1).to(input_dtype),
            "losses": torch.cat(losses, dim=1),
            "grad_norms": grad_norms,
            "past_key_values": None,
        }

    def forward_w_past(self, q, ref_v, chunk_size, loss_mask=None, past_key_values=None):
        """Streaming: queues carried across calls in past_key_values
        (q, hyp_v, ref_v, None, mask, None) (fwmlp.py:299-497)."""
        B, T = q.shape[:2]
        input_dtype = q.dtype
        if self.fp32_fw:
            q, ref_v = q.float(), ref_v.float()
        dev, dt = ref_v.device, ref_v.dtype
        qq = torch.zeros(B, 0, q.size(-1), device=dev, dtype=dt)
        hq = torch.zeros(B, 0, ref_v.size(-1), device=dev, dtype=dt)
        rq = torch.zeros(B, 0, ref_v.size(-1), device=dev, dtype=dt)
        mq = torch.zeros(B, 0, device=dev, dtype=dt) if loss_mask is not None else None
        if past_key_values is not None:
            p_q, p_h, p_r, _, p_m, _ = past_key_values
            if p_h is not None:
                assert p_h.size(1) < chunk_size + self.lookahead, (
                    f"Past key values length {p_h.size(1)} longer than "
                    f"chunk size + lookahead ({chunk_size} + {self.lookahead})."
                )
                qq, hq, rq = torch.cat([p_q, qq], 1), torch.cat([p_h, hq], 1), torch.cat([p_r, rq], 1)
                mq = torch.cat([p_m, mq], 1) if loss_mask is not None else None
        la = self.lookahead
        first = min(chunk_size + la - rq.size(1), T)
        bounds = [(0, first)] + [(s, min(s + chunk_size, T)) for s in range(first, T, chunk_size)]
        updated = False
        params = self.get_fw_named_params()
        outputs, losses, step_grads = [], [], []
        for start, end in bounds:
            cT = end - start
            cq = q[:, start:end].contiguous()
            cmask = loss_mask[:, start:end].contiguous() if loss_mask is not None else None
            hyp = self.retrieve_values(cq, params)["retireved_values"].view(B, cT, -1)
            outputs.append(hyp)
            qq, hq, rq = torch.cat([qq, cq], 1), torch.cat([hq, hyp], 1), torch.cat([rq, ref_v[:, start:end]], 1)
            mq = torch.cat([mq, cmask], 1) if loss_mask is not None else None
            if past_key_values and hq.size(1) < chunk_size:
                continue
            updated = True
            with torch.enable_grad():
                params = {n: p.detach().requires_grad_(True) for n, p in params.items()}
                u_hyp = self.retrieve_values(qq[:, :-la].contiguous(), params)["retireved_values"].contiguous()
                u_mask = mq[:, :-la].contiguous() if mq is not None else None
                u_ref = self._targets(rq).contiguous()
                mem_losses = self.compute_mem_loss(u_hyp.view(-1, u_hyp.size(-1)), u_ref.view(-1, u_ref.size(-1)),
                                                   u_mask.view(-1) if u_mask is not None else None)
                params, grads = self.update_fw(params, mem_losses.mean())
            qq, hq, rq = qq[:, -la:].contiguous(), hq[:, -la:].contiguous(), rq[:, -la:].contiguous()
            mq = mq[:, -la:].contiguous() if u_mask is not None else None
            step_grads.append([g.detach() for g in grads])
            losses.append(mem_losses.view(B, -1).detach())
        grad_norms = None
        if updated:
            with torch.no_grad():
                grad_norms = [torch.stack([g[i].norm() for g in step_grads]).mean() for i in range(len(params))]
                for n, p in self.named_parameters():
                    if n in params:
                        p.data.copy_(params[n].data.to(p.dtype))
        return {
            "output": torch.cat(outputs, dim=1).to(input_dtype),
            "losses": torch.cat(losses, dim=1) if updated else None,
            "grad_norms": grad_norms,
            "past_key_values": (qq, hq, rq, None, mq, None),
        }

    @torch.compiler.disable(recursive=True)
    def forward(self, q, ref_v, chunk_size, loss_mask=None, past_key_values=None):
        if past_key_values is None:
            return self.forward_wo_past(q, ref_v, chunk_size, loss_mask=loss_mask)
        return self.forward_w_past(q, ref_v, chunk_size, loss_mask=loss_mask, past_key_values=past_key_values)


__all__ = ["FastWeightMLP", "l2norm"]
