"""The library's kernel timing (pkm_kernel_timing_*) used by the benchmark:
records appear for the named kernels of each call, including backward passes
that the autograd engine runs on its own thread, carry positive durations,
stop when timing ends, and leave the results unchanged."""
import pytest
import torch

from modelos_amd import _lib
from modelos_amd import embedding_bag as eb
from modelos_amd.pkm.xformer_embeddingbag import xformers_embedding_bag
from tests.helpers import eb_inputs

pytestmark = pytest.mark.gpu


def test_kernel_timing_records_entry_point_kernels():
    dev = torch.device("cuda", 0)
    W, idx, p, g = [t.to(dev) for t in eb_inputs(64, 32, 4096, 256, torch.bfloat16, seed=3)]
    base_out = eb.eb_forward(idx, W, p)
    base_gW, base_gp = eb.eb_backward(idx, W, p, g)
    timer = _lib.KernelTimer()
    with timer:
        outs = [eb.eb_forward(idx, W, p) for _ in range(3)]
        grads = [eb.eb_backward(idx, W, p, g) for _ in range(2)]
    assert len(timer.ms("eb_fwd")) == 3
    assert len(timer.ms("eb_bwd_rows")) == 2
    assert all(ms > 0 for ms in timer.ms("eb_fwd") + timer.ms("eb_bwd_rows"))
    assert timer.ms("score_topk") == []
    for o in outs:
        assert torch.equal(o, base_out)
    for gW, gp in grads:
        assert torch.equal(gW, base_gW) and torch.equal(gp, base_gp)
    # timing is off after the context: a new timer sees only its own calls
    eb.eb_backward(idx, W, p, g)
    with _lib.KernelTimer() as t2:
        pass
    assert t2.ms("eb_bwd_rows") == []


def test_kernel_timing_sees_autograd_thread():
    dev = torch.device("cuda", 0)
    W, idx, p, g = [t.to(dev) for t in eb_inputs(32, 16, 2048, 128, torch.bfloat16, seed=4)]
    W.requires_grad_(True)
    p.requires_grad_(True)
    with _lib.KernelTimer() as timer:
        out = xformers_embedding_bag(idx, W, p)
        out.backward(g)
        torch.cuda.synchronize()
    assert len(timer.ms("eb_fwd")) == 1
    assert len(timer.ms("eb_bwd_rows")) == 1
