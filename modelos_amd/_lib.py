"""ctypes binding of libpkm_hip.so, the C ABI declared in include/pkm_hip.h.

The library is loaded after torch, so it binds to the HIP runtime torch has
already loaded (one runtime per process: streams and device pointers are
shared). A missing library is an error, never a silent fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is opened)

LIB_PATH = Path(os.environ.get("PKM_HIP_LIB", Path(__file__).with_name("libpkm_hip.so")))

# name -> (restype, argtypes); mirrors include/pkm_hip.h
SIGNATURES = {
    "pkm_version": (c_int, []),
    "pkm_last_error_string": (c_char_p, []),
    "pkm_eb_fwd": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p],
    ),
    "pkm_eb_bwd_workspace_size": (c_size_t, [c_int64, c_int64, c_int64, c_int64]),
    "pkm_eb_bwd": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # weight, num_rows, dim, weight_dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_void_p, c_int,  # grad_out, grad_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_void_p,  # grad_weight, grad_psw
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_eb_bwd_prepare": (
        c_int,
        [
            c_int64, c_int64, c_int,  # num_rows, dim, weight_dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_eb_bwd_prepared": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # weight, num_rows, dim, weight_dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_void_p, c_int,  # grad_out, grad_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_void_p,  # grad_weight, grad_psw
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_eb_bwd_accumulate": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # weight, num_rows, dim, weight_dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_void_p, c_int,  # grad_out, grad_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_void_p,  # grad_weight (in / out), grad_psw
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_eb_bwd_noalloc": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # weight, num_rows, dim, weight_dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_void_p, c_int,  # grad_out, grad_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_void_p, c_void_p,  # grad_weight, grad_psw, stream
        ],
    ),
    "pkm_eb_bwd2": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # gbar, num_rows, dim, gbar_dtype
            c_void_p, c_void_p, c_int,  # indices, a, a_dtype
            c_void_p, c_int,  # grad_out, grad_dtype
            c_int64, c_int64,  # bags, bag_size
            c_void_p, c_void_p, c_void_p,  # d_grad_out, d_a, stream
        ],
    ),
    "pkm_count_invalid_indices": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "pkm_score_topk_workspace_size": (c_size_t, [c_int64, c_int64, c_int64, c_int]),
    "pkm_score_topk_ws": (
        c_int,
        [
            c_void_p, c_void_p,  # query, keys
            c_int64, c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, half, knn
            c_int, c_int,  # score_type, dtype
            c_void_p, c_void_p,  # out_scores, out_indices
            c_void_p, c_void_p,  # out_sub_indices1, out_sub_indices2
            c_void_p, c_void_p,  # out_sub_scores1, out_sub_scores2
            c_void_p, c_size_t,  # workspace, workspace_bytes
            c_void_p,  # stream
        ],
    ),
    "pkm_score_topk": (
        c_int,
        [
            c_void_p, c_void_p,  # query, keys
            c_int64, c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, half, knn
            c_int, c_int,  # score_type, dtype
            c_void_p, c_void_p,  # out_scores, out_indices
            c_void_p, c_void_p,  # out_sub_indices1, out_sub_indices2
            c_void_p, c_void_p,  # out_sub_scores1, out_sub_scores2
            c_void_p,  # stream
        ],
    ),
    "pkm_score_grad_dense": (
        c_int,
        [
            c_void_p, c_void_p, c_int,  # indices, d_scores, dtype
            c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, knn
            c_void_p, c_void_p,  # d_sub_scores1, d_sub_scores2
            c_void_p, c_void_p,  # d_sub_dense, stream
        ],
    ),
    "pkm_idw_grad_coef_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "pkm_idw_grad_coef": (
        c_int,
        [
            c_void_p, c_int, c_void_p, c_void_p, c_void_p,  # dS, dtype, qq, kk, dots
            c_int64, c_int64, c_int64,  # batches, tokens, n_keys
            c_void_p, c_void_p, c_void_p,  # U, rowsum, colsum
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_score_grad_sparse_workspace_size": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int64]),
    "pkm_score_grad_sparse": (
        c_int,
        [
            c_void_p, c_void_p, c_int,  # indices, d_scores, dtype
            c_int64, c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, half, knn
            c_void_p, c_void_p, c_void_p, c_void_p,  # query, keys, d_query, d_keys
            c_void_p, c_size_t, c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "pkm_fw_sgd_update": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int,  # values, grad, counts, num_rows, dim, dtype
            c_float, c_float, c_float, c_int,  # scale, lr, weight_decay, grad_clip
            c_void_p, c_void_p, c_void_p,  # scaled_grad, new_values, stream
        ],
    ),
    "pkm_fw_sgd_update_bwd": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p,  # d_new_values, d_scaled_grad, scaled_grad, counts
            c_int64, c_int64, c_int,  # num_rows, dim, dtype
            c_float, c_float, c_float, c_int,  # scale, lr, weight_decay, grad_clip
            c_void_p, c_void_p, c_void_p,  # d_values, d_grad, stream
        ],
    ),
    "pkm_eb_bwd_sgd": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int,  # values, num_rows, dim, dtype
            c_void_p, c_void_p, c_int,  # indices, psw, psw_dtype
            c_void_p, c_int64, c_int64,  # grad_out, bags, bag_size
            c_float, c_float, c_float, c_int,  # scale, lr, weight_decay, grad_clip
            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,  # new_values, scaled_grad, grad_psw, counts, row_sumsq
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_eb_bwd2_sgd": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p,  # d_new_values, d_scaled_grad, scaled_grad, counts
            c_int64, c_int64, c_int,  # num_rows, dim, dtype
            c_float, c_float, c_int,  # scale, lr, grad_clip
            c_void_p, c_void_p, c_int,  # indices, a, a_dtype
            c_void_p, c_int64, c_int64,  # grad_out, bags, bag_size
            c_void_p, c_void_p, c_void_p,  # d_grad_out, d_a, stream
        ],
    ),
    "pkm_me_grad_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "pkm_me_grad_fwd": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p, c_int,  # s1, s2, sel1, sel2, dtype
            c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, topk
            c_int, c_float,  # score_type, weight
            c_void_p, c_void_p, c_void_p,  # qq, kk, dots
            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,  # entropy, coef, avec, pbar, colsum
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_me_grad_hvp": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p, c_int,  # s1, s2, sel1, sel2, dtype
            c_int64, c_int64, c_int64, c_int64,  # num_tokens, heads, n_keys, topk
            c_int, c_float,  # score_type, weight
            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,  # qq, kk, kg, dots, qg
            c_void_p, c_void_p, c_void_p,  # avec, pbar, adot
            c_void_p, c_void_p, c_void_p,  # d_s1, d_s2, ul
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
    "pkm_softmax_fwd": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "pkm_softmax_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "pkm_column_sum_workspace_size": (c_size_t, [c_int64, c_int64]),
    "pkm_column_sum": (c_int, [c_void_p, c_int64, c_int64, c_int, c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "pkm_swilu_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "pkm_swilu_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p]),
    "pkm_rmsnorm_fwd": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int, c_float, c_void_p, c_void_p, c_void_p],
    ),
    "pkm_kernel_timing_begin": (c_int, []),
    "pkm_kernel_timing_read": (c_int, [c_char_p, c_void_p, c_int64, c_void_p]),
    "pkm_kernel_timing_end": (c_int, []),
    "pkm_rmsnorm_bwd_workspace_size": (c_size_t, [c_int64, c_int64]),
    "pkm_rmsnorm_bwd": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p,  # dy, x, weight, rstd
            c_int64, c_int64, c_int,  # rows, dim, dtype
            c_void_p, c_void_p,  # dx, dweight
            c_void_p, c_size_t, c_void_p,  # workspace, bytes, stream
        ],
    ),
}

# pkm_score_t
SCORE_CODES = {"dot": 0, "idw": 1}

# pkm_dtype_t
DTYPE_NONE = -1
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

STATUS_NAMES = {
    1: "invalid argument",
    2: "unsupported",
    3: "workspace too small",
    4: "HIP error",
}


class PkmError(RuntimeError):
    """A libpkm_hip call returned a nonzero status."""

    def __init__(self, fn: str, status: int, message: str):
        self.fn = fn
        self.status = status
        super().__init__(f"{fn} failed ({STATUS_NAMES.get(status, status)}): {message}")


class PkmLibraryMissing(RuntimeError):
    """libpkm_hip.so is not built / not loadable."""


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Opens libpkm_hip.so once and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise PkmLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m modelos_amd.build_lib` "
            "(the PKM lookup path has no CPU fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class CallTimer:
    """Brackets every entry-point call with a pair of timing events on torch's
    current stream (the stream the call enqueues on). Use as a context
    manager; `summary()` synchronises and returns {name: [ms, ...]}."""

    def __init__(self):
        self.events = []

    def __enter__(self):
        global _timer
        self._prev, _timer = _timer, self
        return self

    def __exit__(self, *exc):
        global _timer
        _timer = self._prev
        return False

    def summary(self) -> dict:
        """{(entry point, leading integer arguments): [ms per call]}."""
        torch.cuda.synchronize()
        out: dict = {}
        for key, a, b in self.events:
            out.setdefault(key, []).append(a.elapsed_time(b))
        return out


class KernelTimer:
    """Times single kernels inside multi-kernel entry points with the
    library's own event pairs, recorded on the stream each kernel runs on
    (pkm_kernel_timing_*; process-wide, so backward passes on the autograd
    thread are timed too). Use as a context manager; on exit it synchronises,
    keeps the durations and turns timing off. `ms(kernel)` returns the
    durations of one kernel name in call order."""

    KERNELS = ("eb_fwd", "eb_bwd2", "eb_bwd_rows", "eb_bwd_hot", "score_topk")

    def __init__(self):
        self.records: dict = {}

    def __enter__(self):
        call("pkm_kernel_timing_begin")
        return self

    def __exit__(self, *exc):
        lib = load()
        try:
            for kernel in self.KERNELS:
                count = c_int64(0)
                name = kernel.encode()
                status = lib.pkm_kernel_timing_read(name, None, 0, ctypes.byref(count))
                buf = (c_float * max(count.value, 1))()
                if status == 0 and count.value:
                    status = lib.pkm_kernel_timing_read(name, buf, count.value, ctypes.byref(count))
                if status != 0:
                    raise PkmError("pkm_kernel_timing_read", status,
                                   lib.pkm_last_error_string().decode(errors="replace"))
                self.records[kernel] = list(buf)[: count.value]
        finally:
            lib.pkm_kernel_timing_end()
        return False

    def ms(self, kernel: str) -> list:
        return self.records.get(kernel, [])


_timer: CallTimer | None = None
# positions of the size arguments that name a call's shape in CallTimer keys
_SIZE_ARGS = {
    "pkm_eb_fwd": (1, 2),  # num_rows, dim
    "pkm_eb_bwd": (1, 2),
    "pkm_eb_bwd_noalloc": (1, 2),
    "pkm_eb_bwd_prepare": (0, 1),
    "pkm_eb_bwd_prepared": (1, 2),
    "pkm_eb_bwd_accumulate": (1, 2),
    "pkm_eb_bwd2": (1, 2),
    "pkm_eb_bwd_sgd": (1, 2),
    "pkm_eb_bwd2_sgd": (4, 5),
    "pkm_score_topk": (2, 3, 4, 5),  # num_tokens, heads, n_keys, half
    "pkm_score_topk_ws": (2, 3, 4, 5),
    "pkm_score_grad_sparse": (3, 4, 5, 6),  # num_tokens, heads, n_keys, half
    "pkm_rmsnorm_fwd": (2, 3),  # rows, dim
    "pkm_rmsnorm_bwd": (4, 5),
    "pkm_me_grad_fwd": (5, 6, 7),  # num_tokens, heads, n_keys
    "pkm_me_grad_hvp": (5, 6, 7),
}

# entry points timed under another's name: the workspace form of the scoring
# entry is the same operation (its key pack included)
_TIMED_AS = {"pkm_score_topk_ws": "pkm_score_topk"}



def call(name: str, *args) -> None:
    """Calls an int-status entry point and raises PkmError on failure."""
    lib = load()
    timer = _timer
    if timer is not None:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
    status = getattr(lib, name)(*args)
    if timer is not None:
        end.record()
        key = _TIMED_AS.get(name, name)
        timer.events.append(((key, tuple(args[i] for i in _SIZE_ARGS.get(name, ()))), start, end))
    if status != 0:
        msg = lib.pkm_last_error_string().decode(errors="replace")
        raise PkmError(name, status, msg)


def dtype_code(t: torch.Tensor | None) -> int:
    if t is None:
        return DTYPE_NONE
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype} (float32, bfloat16 and float16 are supported)") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
