"""Compile libttrl_hip.so for gfx950 from tt-rl_amd/csrc, in-tree.

`python -m ttrl_amd._build` (with tt-rl_amd on sys.path) or `build()` from
Python.  Each HIP translation unit is compiled to an object in parallel, then
linked into `ttrl_amd/lib/libttrl_hip.so`, which the package loads at import.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
LIB_DIR = PKG_DIR / "lib"
OBJ_DIR = PKG_DIR.parent / "_build"
LIB_PATH = LIB_DIR / "libttrl_hip.so"

SOURCES = ("runtime.hip", "gemm.hip", "conv_fwd.hip", "conv_dw.hip", "conv_dx.hip", "conv_bwd.hip", "eltwise.hip",
           "heads.hip", "dqn_tail.hip", "optim.hip", "ppo.hip", "act.hip", "rollout.hip", "replay.hip", "gru.hip", "sac_fused.hip")

ARCH = "gfx950"

# Packed-FP32 VALU instructions are disabled on purpose: the compiler may
# still emit scalar and float2 code for them otherwise.
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if not path.exists():
        raise RuntimeError(f"hipcc not found at {path}; a ROCm install is required to build libttrl_hip")
    return str(path)


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_compile, hipcc, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for f in futures:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libttrl_hip.so failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
