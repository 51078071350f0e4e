"""pkm_eb_bwd_noalloc (the embedding-bag backward on the library's fixed
scratch array) against pkm_eb_bwd (the same kernels on a caller workspace),
both called through the C ABI: outputs must be bit-identical (the backward is
deterministic), on two calls in a row, the second with smaller inputs (the
scratch keeps the first call's contents), and too-large sizes must be
rejected with PKM_ERR_WORKSPACE before anything runs."""
import pytest
import torch

from tests.helpers import eb_inputs

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _call_both(W, idx, p, g, device):
    from modelos_amd import _lib
    from modelos_amd import embedding_bag as eb

    W, idx, p, g = (t.to(device) for t in (W, idx, p, g))
    B, L = idx.shape
    K, D = W.shape
    st = _lib.stream_of(device)
    ws_bytes = eb.eb_backward_workspace_bytes(K, D, B, L)
    assert ws_bytes <= SCRATCH_BYTES
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=device)
    ref_gW = torch.empty_like(W)
    ref_gp = torch.empty_like(p)
    _lib.call("pkm_eb_bwd", _lib.ptr(W), K, D, _lib.dtype_code(W), _lib.ptr(idx), _lib.ptr(p), _lib.dtype_code(p),
              _lib.ptr(g), _lib.dtype_code(g), B, L, _lib.ptr(ref_gW), _lib.ptr(ref_gp), _lib.ptr(ws), ws_bytes, st)
    gW = torch.full_like(W, float("nan"))
    gp = torch.full_like(p, float("nan"))
    _lib.call("pkm_eb_bwd_noalloc", _lib.ptr(W), K, D, _lib.dtype_code(W), _lib.ptr(idx), _lib.ptr(p),
              _lib.dtype_code(p), _lib.ptr(g), _lib.dtype_code(g), B, L, _lib.ptr(gW), _lib.ptr(gp), st)
    torch.cuda.synchronize(device)
    return (gW.cpu(), gp.cpu()), (ref_gW.cpu(), ref_gp.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_noalloc_matches_workspace_entry_twice(dtype, device):
    # first call: a fast-weight chunk's shape, with a hot row (heavy-chunk path)
    W, idx, p, g = eb_inputs(4096, 64, 1 << 16, 512, dtype, seed=11)
    idx[:, :5] = 7
    (gW, gp), (rW, rp) = _call_both(W, idx, p, g, device)
    assert torch.equal(gW, rW) and torch.equal(gp, rp), "first call differs from pkm_eb_bwd"
    # second call, smaller: fewer bags, rows and columns than the first left in scratch
    W, idx, p, g = eb_inputs(300, 17, 5000, 256, dtype, seed=12)
    (gW, gp), (rW, rp) = _call_both(W, idx, p, g, device)
    assert torch.equal(gW, rW) and torch.equal(gp, rp), "second (smaller) call differs from pkm_eb_bwd"


def test_noalloc_rejects_sizes_beyond_scratch(device):
    from modelos_amd import _lib

    K, D, B, L = 1 << 20, 1024, 16384, 256  # needs ~248 MiB of workspace
    assert int(_lib.load().pkm_eb_bwd_workspace_size(K, D, B, L)) > SCRATCH_BYTES
    # sizes are checked before any pointer is touched: nothing is launched
    status = _lib.load().pkm_eb_bwd_noalloc(None, K, D, 1, None, None, -1, None, 1, B, L, None, None,
                                            _lib.stream_of(device))
    assert status == 3  # PKM_ERR_WORKSPACE
    msg = _lib.load().pkm_last_error_string().decode()
    assert "scratch" in msg and "pkm_eb_bwd with a workspace" in msg
