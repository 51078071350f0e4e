"""The scoring entry's workspace form (GPU).

pkm_score_topk_ws takes a workspace of the keys' size; where the tile kernel
runs (knn above 32, idw scores, float32, other half widths) it first packs
each block of 16 keys chunk-major into it, so that a k-step's key operands
are one contiguous KB. The operands each lane receives are unchanged, so the
results must equal pkm_score_topk's bit for bit, with every output; the
workspace is rewritten by every call. A workspace that is NULL or too small
gives the unpacked path.
"""
from __future__ import annotations

import pytest
import torch

from modelos_amd import _lib
from oracle import pkm as ref
from tests.helpers import gen

pytestmark = pytest.mark.gpu

# (tokens, heads, n_keys, half, knn, score type, dtype)
CASES = [
    (300, 4, 2048, 256, 64, "dot", torch.bfloat16),  # the large-memory stress shape's kernel (fewer tokens)
    (97, 3, 512, 128, 48, "dot", torch.bfloat16),
    (130, 2, 1024, 64, 32, "idw", torch.bfloat16),
    (70, 5, 256, 96, 16, "dot", torch.float32),
    (65, 2, 2048, 32, 64, "idw", torch.float32),
    (33, 1, 64, 256, 8, "dot", torch.bfloat16),  # half 256, knn 8 bf16 dot: the streaming kernel, packing unused
]


def _ids(c):
    return "N{}-H{}-n{}-h{}-k{}-{}-{}".format(*c[:6], str(c[6]).split(".")[-1])


def _call(entry, q, k, H, n, half, knn, st, ws=None, ws_bytes=0):
    N = q.shape[0]
    dev = q.device
    out = [torch.empty((N * H, knn), dtype=q.dtype, device=dev), torch.empty((N * H, knn), dtype=torch.long, device=dev),
           torch.empty((N, H, knn), dtype=torch.long, device=dev), torch.empty((N, H, knn), dtype=torch.long, device=dev),
           torch.empty((N, H, n), dtype=q.dtype, device=dev), torch.empty((N, H, n), dtype=q.dtype, device=dev)]
    args = [_lib.ptr(q), _lib.ptr(k), N, H, n, half, knn, _lib.SCORE_CODES[st], _lib.dtype_code(q),
            *[_lib.ptr(t) for t in out]]
    if entry == "pkm_score_topk_ws":
        args += [_lib.ptr(ws), ws_bytes]
    _lib.call(entry, *args, _lib.stream_of(dev))
    return out


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_workspace_form_equals_plain_entry(case, device):
    N, H, n, half, knn, st, dt = case
    g = gen(hash(_ids(case)) % 1000)
    q = torch.randn((N, H, 2 * half), generator=g).to(dt).to(device)
    k = (torch.randn((2 * H * n, half), generator=g) / 4).to(dt).to(device)
    need = int(_lib.load().pkm_score_topk_workspace_size(H, n, half, _lib.dtype_code(q)))
    assert need == k.numel() * k.element_size()
    plain = _call("pkm_score_topk", q, k, H, n, half, knn, st)
    ws = torch.full((need,), 0xA5, dtype=torch.uint8, device=device)  # stale contents must not matter
    packed = _call("pkm_score_topk_ws", q, k, H, n, half, knn, st, ws, need)
    # a second call into the same workspace with other keys
    k2 = (torch.randn((2 * H * n, half), generator=g) / 4).to(dt).to(device)
    plain2 = _call("pkm_score_topk", q, k2, H, n, half, knn, st)
    packed2 = _call("pkm_score_topk_ws", q, k2, H, n, half, knn, st, ws, need)
    # a workspace one byte short: the unpacked path
    short = _call("pkm_score_topk_ws", q, k, H, n, half, knn, st, ws, need - 1)
    torch.cuda.synchronize()
    for a, b, c, d, e in zip(plain, packed, plain2, packed2, short):
        assert torch.equal(a, b) and torch.equal(c, d) and torch.equal(a, e)
    if st == "dot" and N * H <= 600:
        # the packed path against the oracle's selection on a few rows
        rows = [0, N // 2, N - 1]
        e_scores, e_idx = ref.get_indices(q[rows].cpu(), k.cpu(), H, knn)[:2]
        got = packed[1].view(N, H, knn)[rows].reshape(-1, knn).cpu()
        assert torch.equal(got, e_idx.reshape(-1, knn))
