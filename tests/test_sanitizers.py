"""Thread- and address-sanitizer builds of the library's host-side native code (CPU only).

``tests/native/host_stress.cpp`` drives the pinned-slab pool, host copy batches and weight-file
read batches (the loader's host staging, run on the shared copy threads) from several threads at
once, plus ``sh_shutdown`` while another thread still copies. ``tests/native/Makefile`` builds it
with the thread sanitizer and with the address and undefined-behaviour sanitizers and runs both;
any race, out-of-bounds access, leak or undefined behaviour fails the run.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

NATIVE = Path(__file__).resolve().parent / "native"
CLANG = Path("/opt/rocm/llvm/bin/clang++")


@pytest.mark.skipif(not CLANG.exists() or shutil.which("make") is None, reason="needs ROCm's clang and make")
def test_host_code_is_clean_under_tsan_and_asan():
    proc = subprocess.run(["make", "-C", str(NATIVE), "run"], capture_output=True, text=True, timeout=600)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert out.count("host_stress: ok (0 failures)") == 2, out[-4000:]
