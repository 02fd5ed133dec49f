"""Builds the native library ``stagehand_amd/_lib/libstagehand_native.so``.

All sources under ``stagehand_amd/csrc`` are compiled by ``hipcc`` for gfx950
into one shared library with a plain C ABI (declared in
``include/stagehand_native.h``). The library is built in-tree so that it
travels with the repository to the GPU machine; nothing is JIT-compiled.

Usage: ``python -m stagehand_amd.build_native`` (or ``build()`` from Python).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libstagehand_native.so"
LIB_PATH = LIB_DIR / LIB_NAME

OFFLOAD_ARCH = "gfx950"
# the HSA runtime (save-back copies on SDMA engines, sh_saveback.cpp)
ROCM_LIB = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
# No fast-math and no denormal flushing: the unpack kernels must round exactly
# as IEEE fp32 does on the host.
# -amdgpu-kernarg-preload-count: gfx950 hands a kernel's first arguments (the unpack kernels'
# six pointers) to every wavefront in SGPRs, so a workgroup's first scalar load (its tile-map
# entry) does not wait for a load of the argument block. Measured on the config-2 cast: +0.2-0.3%.
HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=6",
    "-fno-gpu-rdc",
]


def hipcc_path() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build stagehand_amd")
    return cand


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip")) + sorted(CSRC_DIR.glob("*.cpp"))


def build(verbose: bool = False) -> Path:
    """Compile every native source into ``LIB_PATH`` (always rebuilds)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}",
           *[str(s) for s in sources()], "-o", str(tmp), "-lpthread", f"-L{ROCM_LIB}", "-lhsa-runtime64"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
