"""The native library leaves nothing to the process's exit (CPU only).

Under ``rocprofv3 --memory-copy-trace`` a process that had used the library used to end with a
segmentation fault in ``__cxa_finalize``, after its last line. A library leaves code to that
phase through the handlers it registers with ``__cxa_atexit`` (static destructors, ``atexit``
calls, and the module destructor that the HIP compiler emits for every ``.hip`` translation unit,
which unregisters its fat binary from the HIP runtime) and ``__cxa_thread_atexit_impl`` (C++
``thread_local`` destructors). ``tests/native/exit_probe.c`` interposes both, loads the library,
drives the entry points that run without a GPU on two threads, calls ``sh_shutdown`` and exits;
this test asserts that none of the handlers registered in that whole run, the exit included,
belongs to the library. The kernels live in embedded code objects loaded with the HIP module API
(``csrc/sh_kernels.cpp``), so no fat binary is registered at all.

The reference's native engines end in their Rust ``Drop`` impls when Python drops them
(``turbo_src/engine.rs:395-422``, ``vmm_src/allocator.rs:648-713``); here the same teardown is
``sh_shutdown`` and each object's destroy call.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from stagehand_amd import _native

REPO = Path(__file__).resolve().parent.parent
PROBE = REPO / "tests" / "native" / "exit_probe.c"


@pytest.fixture(scope="module")
def probe(tmp_path_factory) -> Path:
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    _native.lib()  # the library must be built
    out = tmp_path_factory.mktemp("exit_probe") / "exit_probe"
    lib_dir = _native.LIB_PATH.parent
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-rdynamic", f"-I{REPO / 'include'}", str(PROBE), "-o", str(out),
           f"-L{lib_dir}", f"-Wl,-rpath,{lib_dir}", "-lstagehand_native", "-ldl", "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return out


def test_library_registers_no_exit_handlers(probe, tmp_path):
    proc = subprocess.run([str(probe), str(tmp_path / "scratch.bin")], capture_output=True, text=True, timeout=120)
    out = proc.stdout + proc.stderr
    assert "exit_probe: 0 failures" in out, out
    assert "exit_probe: 0 library exit handlers" in out, out
    assert proc.returncode == 0, out


def test_library_registers_no_fat_binary():
    """No undefined reference to the HIP runtime's fat-binary registration: the compiler-emitted
    module constructor and destructor call those."""
    proc = subprocess.run(["nm", "-D", "--undefined-only", str(_native.LIB_PATH)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    names = {line.split()[-1] for line in proc.stdout.splitlines() if line.strip()}
    assert not {n for n in names if "RegisterFatBinary" in n or "RegisterFunction" in n or "RegisterVar" in n}
    assert "__cxa_thread_atexit_impl" not in names
