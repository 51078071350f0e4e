"""FwPKM fast-weight value update: CPU restatement (test infrastructure only).

Semantics (FastWeightProductKeyMemory.update_fw, fwpkm/fwpkm.py:334-365, the
"values" parameter, and update_fw_param at fwpkm.py:266-272, optimizer "sgd"),
as the reference's ATen ops on tensors of the value dtype:

  g = g * scale                                   scale = num_samples * v_dim * topk * heads
  c = bincount(indices, minlength=size).to(dtype); c[c == 0] = 1
  g = g / c[:, None]                              (the returned, unclipped gradient)
  gc = clamp(g, -1, 1) if grad_clip else g
  new = p - lr * (gc + wd * p)

Pinned in tests/test_oracle_fw_update.py against closed forms (no clip and
no decay: new = p - lr * scale * g / count; rows never indexed divide by 1)
and a brute-force count.
"""
from __future__ import annotations

from typing import Tuple

import torch


def row_counts(indices: torch.Tensor, size: int) -> torch.Tensor:
    """bincount of the flattened indices, int64 [size] (fwpkm.py:342)."""
    return torch.bincount(indices.reshape(-1), minlength=size)


def sgd_value_update(p: torch.Tensor, g: torch.Tensor, indices: torch.Tensor, scale: float, lr: float, wd: float,
                     grad_clip: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(new values, scaled unclipped gradient), both in p's dtype."""
    g = g * scale
    binc = row_counts(indices, p.shape[0]).to(g.dtype)
    binc[binc == 0] = 1.0
    g = g / binc.unsqueeze(-1)
    gc = torch.clamp(g, min=-1.0, max=1.0) if grad_clip else g
    dp = lr * (gc + wd * p)
    return p - dp, g
