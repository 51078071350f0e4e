"""Host side of the weighted embedding bag: torch tensors in, HIP kernels run.

Functions here validate shapes/dtypes, allocate outputs with torch's caching
allocator on the inputs' device, and call libpkm_hip.so on torch's current
stream (no host synchronisation). They are the building blocks of the
drop-in autograd functions in modelos_amd.pkm / modelos_amd.fwpkm.

There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def _require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"PKM HIP kernels need ROCm device tensors, got a tensor on {t.device} "
                "(this implementation has no CPU path)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    assert dev is not None
    return dev


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels read rows with 16-byte loads)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _grad_in_own_dtype(grad: torch.Tensor, table_dtype: torch.dtype) -> torch.Tensor:
    """The upstream gradient as the kernels read it: in its own dtype when
    that is the table's or float32 (a float32 gradient of a 16-bit table is
    read as float32, as the reference's kernels widen it,
    pkm/xformer_embeddingbag.py:322); any other dtype as float32 (exact for
    the 16-bit types)."""
    if grad.dtype == table_dtype or grad.dtype == torch.float32:
        return grad
    return grad.float()


def _check_bag_inputs(indices: torch.Tensor, table: torch.Tensor, psw: Optional[torch.Tensor], fn: str) -> None:
    if indices.dtype != torch.long:
        raise TypeError(f"{fn}: indices must be int64 (torch.long), got {indices.dtype}")
    if indices.dim() != 2:
        raise ValueError(f"{fn}: indices must be [bags, bag_size], got shape {tuple(indices.shape)}")
    if table.dim() != 2:
        raise ValueError(f"{fn}: table must be [num_rows, dim], got shape {tuple(table.shape)}")
    if psw is not None and psw.shape != indices.shape:
        raise ValueError(
            f"{fn}: per_sample_weights shape {tuple(psw.shape)} != indices shape {tuple(indices.shape)}"
        )


def eb_forward(
    indices: torch.Tensor, weight: torch.Tensor, per_sample_weights: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """out[b, :] = sum_j psw[b, j] * weight[indices[b, j], :], in weight.dtype.

    float32 accumulation in j order (pkm/xformer_embeddingbag.py:97-113).
    """
    _check_bag_inputs(indices, weight, per_sample_weights, "eb_forward")
    dev = _require_device(indices, weight, per_sample_weights)
    indices = indices.contiguous()
    weight = _aligned(weight)
    psw = per_sample_weights.contiguous() if per_sample_weights is not None else None
    B, L = indices.shape
    K, D = weight.shape
    out = torch.empty((B, D), dtype=weight.dtype, device=dev)
    _lib.call(
        "pkm_eb_fwd",
        _lib.ptr(weight), K, D, _lib.dtype_code(weight),
        _lib.ptr(indices), _lib.ptr(psw), _lib.dtype_code(psw),
        B, L, _lib.ptr(out), _lib.stream_of(dev),
    )
    return out


def eb_backward_workspace_bytes(num_rows: int, dim: int, bags: int, bag_size: int) -> int:
    return int(_lib.load().pkm_eb_bwd_workspace_size(num_rows, dim, bags, bag_size))


_side_streams: dict = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """One extra stream per device (default priority) for work that runs beside
    the current stream."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side_streams.get(key)
    if st is None:
        st = torch.cuda.Stream(device=key)
        _side_streams[key] = st
    return st


class BackwardPrep:
    """The lookup-only part of the backward (sort, row offsets, metadata),
    computed ahead by eb_backward_prepare: its workspace, the sizes it was made
    for, and the event that marks it done."""

    def __init__(self, workspace: torch.Tensor, ws_bytes: int, key: tuple, done: torch.cuda.Event):
        self.workspace, self.ws_bytes, self.key, self.done = workspace, ws_bytes, key, done


def _prep_key(indices, weight, psw) -> tuple:
    """What a prepared workspace depends on: the lookups' storage, shape and
    version counter (an in-place write to indices or psw after the prepare
    changes the version), the table shape and dtype, psw's storage and dtype."""
    return (indices.data_ptr(), tuple(indices.shape), indices._version, tuple(weight.shape), weight.dtype,
            psw.data_ptr() if psw is not None else 0, psw.dtype if psw is not None else None,
            psw._version if psw is not None else 0)


def eb_backward_prepare(
    indices: torch.Tensor, weight: torch.Tensor, per_sample_weights: Optional[torch.Tensor]
) -> BackwardPrep:
    """Runs pkm_eb_bwd_prepare for these lookups on a side stream, after the
    work already queued on the current stream, and returns the handle that
    eb_backward(prepared=...) consumes. indices / psw must stay unchanged until
    then (autograd's saved tensors)."""
    _check_bag_inputs(indices, weight, per_sample_weights, "eb_backward_prepare")
    dev = _require_device(indices, weight, per_sample_weights)
    if not (indices.is_contiguous() and (per_sample_weights is None or per_sample_weights.is_contiguous())):
        raise ValueError("eb_backward_prepare: indices and per_sample_weights must be contiguous")
    B, L = indices.shape
    K, D = weight.shape
    psw = per_sample_weights
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev)
    side.wait_stream(main)
    ws_bytes = eb_backward_workspace_bytes(K, D, B, L)
    with torch.cuda.stream(side):
        workspace = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        _lib.call(
            "pkm_eb_bwd_prepare",
            K, D, _lib.dtype_code(weight),
            _lib.ptr(indices), _lib.ptr(psw), _lib.dtype_code(psw),
            B, L, _lib.ptr(workspace), ws_bytes, side.cuda_stream,
        )
        done = torch.cuda.Event()
        done.record(side)
    # the side stream read these: their memory is not reused before it is done
    indices.record_stream(side)
    if psw is not None:
        psw.record_stream(side)
    return BackwardPrep(workspace, ws_bytes, _prep_key(indices, weight, psw), done)


def eb_backward(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: Optional[torch.Tensor],
    grad_output: torch.Tensor,
    prepared: Optional[BackwardPrep] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Deterministic backward: (grad_weight [K, D] dense in weight.dtype,
    grad_psw [B, L] in psw.dtype or None when psw is None).

    Same outputs as embedding_bag_bw_rev_indices (pkm/xformer_embeddingbag.py:331-386).
    With `prepared` (eb_backward_prepare of the same indices, weight shape and
    psw) only the reduction runs here; the results are bit-identical.
    """
    _check_bag_inputs(indices, weight, per_sample_weights, "eb_backward")
    dev = _require_device(indices, weight, per_sample_weights, grad_output)
    B, L = indices.shape
    K, D = weight.shape
    if grad_output.shape != (B, D):
        raise ValueError(f"eb_backward: grad_output shape {tuple(grad_output.shape)} != {(B, D)}")
    indices = indices.contiguous()
    weight = _aligned(weight)
    psw = per_sample_weights.contiguous() if per_sample_weights is not None else None
    grad_output = _aligned(_grad_in_own_dtype(grad_output, weight.dtype))
    grad_weight = torch.empty_like(weight, memory_format=torch.contiguous_format)
    grad_psw = torch.empty_like(psw, memory_format=torch.contiguous_format) if psw is not None else None
    args = (
        _lib.ptr(weight), K, D, _lib.dtype_code(weight),
        _lib.ptr(indices), _lib.ptr(psw), _lib.dtype_code(psw),
        _lib.ptr(grad_output), _lib.dtype_code(grad_output),
        B, L,
        _lib.ptr(grad_weight), _lib.ptr(grad_psw),
    )
    if prepared is not None:
        if prepared.key != _prep_key(indices, weight, psw):
            raise ValueError(
                "eb_backward: `prepared` was made for other lookups or another table shape, "
                "or indices / per_sample_weights were modified in place since"
            )
        main = torch.cuda.current_stream(dev)
        main.wait_event(prepared.done)
        prepared.workspace.record_stream(main)
        _lib.call("pkm_eb_bwd_prepared", *args, _lib.ptr(prepared.workspace), prepared.ws_bytes,
                  _lib.stream_of(dev))
        return grad_weight, grad_psw
    ws_bytes = eb_backward_workspace_bytes(K, D, B, L)
    workspace = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    _lib.call("pkm_eb_bwd", *args, _lib.ptr(workspace), ws_bytes, _lib.stream_of(dev))
    return grad_weight, grad_psw


def eb_backward_into(
    indices: torch.Tensor,
    weight: torch.Tensor,
    per_sample_weights: Optional[torch.Tensor],
    grad_output: torch.Tensor,
    grad_weight: torch.Tensor,
) -> Optional[Tuple[torch.Tensor, Optional[torch.Tensor]]]:
    """eb_backward adding the table gradient into `grad_weight` in place
    (pkm_eb_bwd_accumulate): grad_weight + eb_backward(...)[0], bit for bit,
    without a separate add over the table. Returns (grad_weight, grad_psw),
    or None, with nothing done, where the kernels have no accumulating path
    (a gradient dtype other than the table's, rows narrower than 64 lanes, a
    grad_weight that is not a contiguous aligned [K, D] of the table's dtype)."""
    _check_bag_inputs(indices, weight, per_sample_weights, "eb_backward_into")
    dev = _require_device(indices, weight, per_sample_weights, grad_output, grad_weight)
    B, L = indices.shape
    K, D = weight.shape
    if grad_output.shape != (B, D):
        raise ValueError(f"eb_backward_into: grad_output shape {tuple(grad_output.shape)} != {(B, D)}")
    if (grad_weight.shape != weight.shape or grad_weight.dtype != weight.dtype or not grad_weight.is_contiguous()
            or grad_weight.data_ptr() % 16 or grad_output.dtype != weight.dtype):
        return None
    indices = indices.contiguous()
    weight = _aligned(weight)
    psw = per_sample_weights.contiguous() if per_sample_weights is not None else None
    grad_output = _aligned(grad_output)
    grad_psw = torch.empty_like(psw, memory_format=torch.contiguous_format) if psw is not None else None
    ws_bytes = eb_backward_workspace_bytes(K, D, B, L)
    workspace = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    try:
        _lib.call("pkm_eb_bwd_accumulate", _lib.ptr(weight), K, D, _lib.dtype_code(weight), _lib.ptr(indices),
                  _lib.ptr(psw), _lib.dtype_code(psw), _lib.ptr(grad_output), _lib.dtype_code(grad_output), B, L,
                  _lib.ptr(grad_weight), _lib.ptr(grad_psw), _lib.ptr(workspace), ws_bytes, _lib.stream_of(dev))
    except _lib.PkmError as e:
        if e.status == 2:  # PKM_ERR_UNSUPPORTED: checked before anything is enqueued
            return None
        raise
    return grad_weight, grad_psw


def eb_double_backward(
    indices: torch.Tensor,
    a: Optional[torch.Tensor],
    grad_output: torch.Tensor,
    g_bar: torch.Tensor,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """VJP of grad_weight = EBbwd(indices, a, grad_output) given g_bar = dL/d(grad_weight):
    (d_grad_output [B, D], d_a [B, L] or None).

    Same outputs as EmbeddingBagBW.backward
    (fwpkm/xformer_embeddingbag_grad_wrapper.py:42-74).
    """
    _check_bag_inputs(indices, g_bar, a, "eb_double_backward")
    dev = _require_device(indices, a, grad_output, g_bar)
    B, L = indices.shape
    K, D = g_bar.shape
    if grad_output.shape != (B, D):
        raise ValueError(f"eb_double_backward: grad_output shape {tuple(grad_output.shape)} != {(B, D)}")
    indices = indices.contiguous()
    out_dtype = grad_output.dtype
    # g_bar [K, D] is read in its own dtype (no copy of it); grad_output [B, D] in its own dtype when
    # that is g_bar's or float32, else as float32 (the reference's type promotion computes in the
    # wider type; autograd hands the result back in grad_output's dtype)
    g_bar = _aligned(g_bar)
    g = _aligned(_grad_in_own_dtype(grad_output, g_bar.dtype))
    if g_bar.dtype == torch.float32 and g.dtype != torch.float32:
        g = g.float()
    a = a.contiguous() if a is not None else None
    d_grad_output = torch.empty((B, D), dtype=g.dtype, device=dev)
    d_a = torch.empty_like(a, memory_format=torch.contiguous_format) if a is not None else None
    _lib.call(
        "pkm_eb_bwd2",
        _lib.ptr(g_bar), K, D, _lib.dtype_code(g_bar),
        _lib.ptr(indices), _lib.ptr(a), _lib.dtype_code(a),
        _lib.ptr(g), _lib.dtype_code(g),
        B, L,
        _lib.ptr(d_grad_output), _lib.ptr(d_a), _lib.stream_of(dev),
    )
    return d_grad_output.to(out_dtype), d_a


def count_invalid_indices(indices: torch.Tensor, num_rows: int) -> int:
    """Number of entries outside [0, num_rows) (synchronises)."""
    dev = _require_device(indices)
    indices = indices.contiguous()
    out = torch.empty((1,), dtype=torch.int64, device=dev)
    _lib.call(
        "pkm_count_invalid_indices",
        _lib.ptr(indices), indices.numel(), num_rows, _lib.ptr(out), _lib.stream_of(dev),
    )
    return int(out.item())
