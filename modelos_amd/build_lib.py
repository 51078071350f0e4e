"""Builds libpkm_hip.so (the C-ABI library of HIP kernels) in-tree for gfx950.

Usage: python -m modelos_amd.build_lib [--jobs N]

Each csrc/*.hip file is compiled to an object under modelos_amd/_build/ in
parallel, then linked into modelos_amd/libpkm_hip.so. Always rebuilds.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libpkm_hip.so"
INCLUDE_DIR = PKG_DIR.parent / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: hipcc would otherwise fuse pairs of float ops into
# v_pk_{add,mul,fma}_f32, which are kept out of this library on purpose.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]


# Per-source flags. eb_bwd.hip: its atomics are issued by one lane on purpose
# and their results are used late (ticket counters taken ahead of use); the
# atomic optimizer would rewrite each into a wave-wide form whose result is
# read right after the atomic, a wait for every load in flight.
# score_topk.hip: MFMA accumulators in arch VGPRs, where the score words are
# packed from them (in AGPRs each element costs a copy out first).
SOURCE_FLAGS = {
    "eb_bwd.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
    "score_topk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    """Compiles every csrc/*.hip and links libpkm_hip.so; returns its path."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the PKM HIP library cannot be built")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)


if __name__ == "__main__":
    main()
