"""Process teardown: no native thread of the library outlives ``_native.shutdown``.

The reference's Rust engines stop their threads and free their streams, events and pinned
memory in their ``Drop`` impls (turbo_src/engine.rs:395-422, vmm_src/allocator.rs:648-713,
vmm_src/prefetch.rs:22-46). Here every object that owns native state is registered for an
ordered close at interpreter exit, and ``sh_shutdown`` then joins the shared host copy threads,
so nothing of the library still runs when the HIP runtime and the profiler's tools tear down.
Each case runs in a child process, counts the threads named ``sh-*`` from
``/proc/self/task``, and exits through the atexit path with status 0.
"""
from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent

PRELUDE = textwrap.dedent("""
    import os, sys
    sys.path.insert(0, {repo!r})

    def sh_threads():
        names = []
        for tid in os.listdir("/proc/self/task"):
            try:
                with open(f"/proc/self/task/{{tid}}/comm") as f:
                    names.append(f.read().strip())
            except OSError:
                pass
        return sorted(n for n in names if n.startswith("sh-"))
""")


def _run_child(body: str, timeout: int = 300) -> str:
    code = PRELUDE.format(repo=str(REPO)) + textwrap.dedent(body)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=timeout)
    assert proc.returncode == 0, f"child exited {proc.returncode}\nstdout:\n{proc.stdout}\nstderr:\n{proc.stderr}"
    return proc.stdout


def test_host_threads_end_at_shutdown_and_at_exit(tmp_path):
    """Host-only objects: an unpinned pool, host copy batches and a weight file read on the copy
    threads. ``shutdown`` closes them and joins the copy threads; the library works again after
    it, and the atexit path ends the second set of threads too."""
    data = tmp_path / "w.bin"
    data.write_bytes(bytes(range(256)) * 4096 * 16)
    out = _run_child(f"""
        import ctypes, numpy as np, torch
        from stagehand_amd import _native
        from stagehand_amd.pool import PinnedPool
        from stagehand_amd.fileio import WeightFile
        assert sh_threads() == []
        pool = PinnedPool(total_mb=8, slab_mb=4, alignment=512, pinned=False)
        src = torch.arange(64 << 20, dtype=torch.uint8)
        dst = torch.empty_like(src)
        items = np.zeros(1, dtype=_native.COPY_ITEM_DTYPE)
        items[0] = (dst.data_ptr(), src.data_ptr(), src.numel())
        _native.call("sh_host_copy_batch", items.ctypes.data, 1, 8)
        assert torch.equal(dst, src)
        wf = WeightFile({str(data)!r})
        buf = torch.empty(wf.size, dtype=torch.uint8)
        wf.read_into(buf, 0)
        assert bytes(buf[:256].tolist()) == bytes(range(256))
        running = sh_threads()
        assert running and all(n == "sh-copy" for n in running), running
        left = _native.shutdown()
        assert all(v == 0 for v in left.values()), left
        assert sh_threads() == [], sh_threads()
        assert pool.handle is None  # closed by the shutdown
        _native.call("sh_host_copy_batch", items.ctypes.data, 1, 8)  # starts the copy threads again
        assert sh_threads()
        print("threads", len(running), "ok")
    """)
    assert "ok" in out


@pytest.mark.gpu
def test_device_workers_end_at_shutdown(tmp_path):
    """Every kind of native worker: a block loader (worker and advisor threads), an SDMA
    save-back engine, a turbo engine (its write-back engine), a VMM allocator (prefetch worker)
    and the copy threads. After ``shutdown`` none is left, every native object is destroyed, and
    the process exits with status 0."""
    out = _run_child("""
        import numpy as np, torch
        from stagehand_amd import _native
        from stagehand_amd.pool import PinnedPool
        from stagehand_amd.transfer import AsyncTransferEngine, BlockSource
        from stagehand_amd.turbo import TransferEngine
        from stagehand_amd.vmm import SlabAllocator
        torch.cuda.init()
        torch.zeros(1, device="cuda").add_(1)
        torch.cuda.synchronize()
        assert sh_threads() == []
        pool = PinnedPool(total_mb=8, slab_mb=4, alignment=512)
        eng = AsyncTransferEngine(pool, save_back="sdma")
        host = torch.randint(0, 256, (3 << 20,), dtype=torch.uint8)
        dst = torch.zeros(host.numel(), dtype=torch.uint8, device="cuda")
        eng.wait(eng.submit_block_load("b0", BlockSource([(0, host)], host.numel()), dst))
        home = torch.zeros(host.numel(), dtype=torch.uint8, pin_memory=True)
        eng.d2h_into(dst, home).synchronize()
        assert torch.equal(home, host)
        turbo = TransferEngine()
        turbo.register_block([4096, 8192])
        turbo.initialize(torch.cuda.current_device(), 3)
        vmm = SlabAllocator(device=torch.cuda.current_device())
        import time
        roles = ("sh-loader", "sh-advisor", "sh-saveback", "sh-vmm-prefetch", "sh-copy")
        deadline = time.monotonic() + 10.0
        while True:  # a thread names itself as its first action: give new ones a moment
            running = sh_threads()
            if all(r in running for r in roles) or time.monotonic() > deadline:
                break
            time.sleep(0.01)
        for role in roles:
            assert role in running, (role, running)
        left = _native.shutdown()
        assert all(v == 0 for v in left.values()), left
        assert sh_threads() == [], sh_threads()
        print("roles", sorted(set(running)), "ok", flush=True)
    """)
    assert "ok" in out
