"""The C-ABI library loads, exports every entry point include/pkm_hip.h
declares, and rejects bad arguments with status codes before touching a GPU.
CPU only: no call here launches a kernel."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pkm_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(pkm_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from modelos_amd import _lib

    if not _lib.LIB_PATH.exists():
        from modelos_amd import build_lib

        build_lib.build(verbose=False)
    return _lib.load()


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ["pkm_eb_fwd", "pkm_eb_bwd", "pkm_eb_bwd2", "pkm_eb_bwd_workspace_size", "pkm_last_error_string"]:
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_signatures_cover_the_header():
    from modelos_amd import _lib

    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_version(lib):
    assert lib.pkm_version() >= 1


def test_invalid_arguments_return_status(lib):
    from modelos_amd import _lib

    # bad weight dtype
    st = lib.pkm_eb_fwd(None, 10, 8, 7, None, None, -1, 4, 2, None, None)
    assert st == 1
    assert b"dtype" in lib.pkm_last_error_string()
    # psw pointer given with dtype NONE
    st = lib.pkm_eb_fwd(None, 10, 8, 1, None, ctypes.c_void_p(16), -1, 4, 2, ctypes.c_void_p(16), None)
    assert st == 1
    # negative sizes
    st = lib.pkm_eb_fwd(None, -1, 8, 1, None, None, -1, 4, 2, None, None)
    assert st == 1
    # zero bags: nothing to do, no kernel
    assert lib.pkm_eb_fwd(None, 10, 8, 1, None, None, -1, 0, 2, None, None) == 0
    # backward: the gradient must be of the weight's dtype or float32 (a bf16 gradient of a float32 table)
    st = lib.pkm_eb_bwd(None, 10, 8, 0, None, None, -1, None, 1, 4, 2, None, None, None, 0, None)
    assert st == 2
    # backward: unsupported row length for the dot-product kernels
    st = lib.pkm_eb_bwd(
        ctypes.c_void_p(16), 10, 24, 1, ctypes.c_void_p(16), None, -1, ctypes.c_void_p(16), 1, 4, 2,
        ctypes.c_void_p(16), None, ctypes.c_void_p(256), 1 << 30, None,
    )
    assert st == 2, _lib.load().pkm_last_error_string()
    # backward: workspace too small
    st = lib.pkm_eb_bwd(
        ctypes.c_void_p(16), 10, 8, 1, ctypes.c_void_p(16), None, -1, ctypes.c_void_p(16), 1, 4, 2,
        ctypes.c_void_p(16), None, ctypes.c_void_p(256), 16, None,
    )
    assert st == 3
    # double backward: a bf16 upstream gradient beside a float32 gbar
    st = lib.pkm_eb_bwd2(None, 10, 8, 0, None, None, -1, None, 1, 4, 2, None, None, None)
    assert st == 2


def test_workspace_size_grows_with_problem(lib):
    small = lib.pkm_eb_bwd_workspace_size(1000, 64, 10, 8)
    big = lib.pkm_eb_bwd_workspace_size(1 << 20, 1024, 16384, 128)
    assert 0 < small < big
    assert lib.pkm_eb_bwd_workspace_size(-1, 64, 10, 8) == 0
    # dominated by sort buffers (16 B / lookup) and the heavy-row partials (8*D/256 B / lookup)
    N = 16384 * 128
    assert big >= 16 * N + (2 * N // 256) * 1024 * 4


def test_python_wrappers_reject_cpu_tensors():
    import torch

    from modelos_amd import embedding_bag as eb

    W = torch.zeros(4, 8)
    idx = torch.zeros(2, 3, dtype=torch.long)
    with pytest.raises(RuntimeError, match="no CPU path"):
        eb.eb_forward(idx, W, None)
    with pytest.raises(TypeError):
        eb.eb_forward(idx.int(), W, None)
    with pytest.raises(ValueError):
        eb.eb_forward(idx, W, torch.zeros(3, 2))
