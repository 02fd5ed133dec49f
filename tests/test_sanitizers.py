"""Thread- and address-sanitizer builds of the library's host-side native code (CPU only).

``tests/native/host_stress.cpp`` drives the pinned-slab pool, host copy batches and weight-file
read batches (the loader's host staging, run on the shared copy threads) from several threads at
once, plus ``sh_shutdown`` while another thread still copies.

``tests/native/engine_stress.cpp`` drives the threaded engines themselves: the block loader
(overlapping tickets finished in any order, zero-byte tickets, file ranges, pinned pieces behind
a save-back ticket, digests), the save-back engine (submits on one thread, waits and releases on
another, changed-chunk copies, destroy with queued tickets), the turbo engine (write-backs in
changed chunks, deferred look-ahead copies, injected copy failures) and the VMM allocator
(ensure/release on three threads against eviction, prefetch and priority changes on a fourth).
It links every host source of the library against ``tests/native/fake_hip.cpp``, a CPU stand-in
for the HIP and HSA calls with the runtime's ordering rules (streams are worker threads, events
complete when their stream reaches them, SDMA copies run on an engine thread), so the sanitizers
see the engines' real threads and hand-offs without a GPU. The reference's protocols they cover:
``vmm_src/allocator.rs:227-273``, ``vmm_src/eviction.rs:50-78``, ``vmm_src/prefetch.rs:22-46``,
``turbo_src/engine.rs:202-341``.

``tests/native/Makefile`` builds both programs with the thread sanitizer and with the address and
undefined-behaviour sanitizers and runs all four; any race, out-of-bounds access, leak, undefined
behaviour or wrong byte fails the run.
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
    proc = subprocess.run(["make", "-C", str(NATIVE), "run"], capture_output=True, text=True, timeout=900)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert out.count("host_stress: ok (0 failures)") == 2, out[-4000:]
    assert out.count("engine_stress: ok (0 failures)") == 2, out[-4000:]
