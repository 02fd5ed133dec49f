"""The SDMA save-back engine (native ``sh_saveback``) and the transfer engine's use of it.

Save-back copies move evicted blocks' device bytes into pinned host memory (the
reference's synchronous ``param.data.to("cpu")``, src/stagehand/scheduler.py:1216-1226).
Here they run on a system DMA engine: ordered after the work queued on a stream
before the submit, completing in submission order, and waited for by the loader
when a load reads what they wrote. Every case checks bytes bit for bit.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from stagehand_amd import _native
from stagehand_amd._native import COPY_ITEM_DTYPE
from stagehand_amd.pool import PinnedPool
from stagehand_amd.transfer import AsyncTransferEngine, BlockSource, NativeEvent, SaveBackEngine, SaveBackTicket

pytestmark = pytest.mark.gpu


def _items(pairs: list[tuple[torch.Tensor, torch.Tensor]]) -> np.ndarray:
    items = np.zeros(len(pairs), dtype=COPY_ITEM_DTYPE)
    for i, (dst, src) in enumerate(pairs):
        items[i] = (dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size())
    return items


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def test_copies_land_bit_exact():
    """Sizes from one byte to tens of MiB, odd lengths and offsets, several copies per ticket."""
    g = torch.Generator(device="cuda").manual_seed(1)
    sizes = [1, 15, 4096, 4097, (1 << 20) + 3, (48 << 20) + 5]
    srcs = [torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g) for n in sizes]
    dsts = [torch.zeros(n + 7, dtype=torch.uint8, pin_memory=True)[3:3 + n] for n in sizes]
    sb = SaveBackEngine(torch.cuda.current_device())
    one = sb.submit(_items([(dsts[0], srcs[0])]), _stream())
    rest = sb.submit(_items(list(zip(dsts[1:], srcs[1:]))), _stream())
    rest.synchronize()
    assert one.query() and rest.query()
    for d, s in zip(dsts, srcs):
        assert torch.equal(d, s.cpu())
    sb.close()


def test_copies_read_what_the_stream_wrote_before_the_submit():
    """The submit is issued while kernels that produce the source are still queued: the copy
    waits for them (the worker waits for the event recorded at submit)."""
    n = 32 << 20
    a = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
    src = torch.zeros(n, dtype=torch.uint8, device="cuda")
    dst = torch.zeros(n, dtype=torch.uint8, pin_memory=True)
    sb = SaveBackEngine(torch.cuda.current_device())
    for rep in range(3):
        torch.cuda.synchronize()
        y = a
        for _ in range(12):  # keep the stream busy for a while
            y = (y @ a) * 1e-3
        src.copy_(y.view(torch.uint8).reshape(-1)[:n])
        src.add_(rep + 1)
        t = sb.submit(_items([(dst, src)]), _stream())
        t.synchronize()
        torch.cuda.synchronize()
        assert torch.equal(dst, src.cpu()), rep
    sb.close()


def test_tickets_complete_in_order_release_and_errors():
    g = torch.Generator(device="cuda").manual_seed(2)
    srcs = [torch.randint(0, 256, (8 << 20,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(3)]
    dsts = [torch.zeros(8 << 20, dtype=torch.uint8, pin_memory=True) for _ in range(3)]
    sb = SaveBackEngine(torch.cuda.current_device())
    tickets = [sb.submit(_items([(d, s)]), _stream()) for d, s in zip(dsts, srcs)]
    tickets[-1].synchronize()  # covers the earlier tickets
    for d, s in zip(dsts, srcs):
        assert torch.equal(d, s.cpu())
    assert all(t.query() for t in tickets)
    lib, h = _native.lib(), sb.handle
    assert lib.sh_saveback_release(h, tickets[0].ticket) == _native.SH_OK
    assert lib.sh_saveback_release(h, tickets[0].ticket) == _native.SH_OK  # twice: a no-op
    assert lib.sh_saveback_query(h, 10**9) == _native.SH_ERR_INVALID
    with pytest.raises(ValueError):
        _native.call("sh_saveback_wait", h, 0)
    bad = np.zeros(1, dtype=COPY_ITEM_DTYPE)
    bad[0] = (0, srcs[0].data_ptr(), 16)
    with pytest.raises(ValueError):
        sb.submit(bad, _stream())
    empty = sb.submit(np.zeros(0, dtype=COPY_ITEM_DTYPE), _stream())
    empty.synchronize()
    sb.close()
    assert tickets[1].query()  # a closed engine waited for every copy
    tickets[1].synchronize()


def test_close_issues_and_waits_for_queued_copies():
    g = torch.Generator(device="cuda").manual_seed(3)
    src = torch.randint(0, 256, (96 << 20,), dtype=torch.uint8, device="cuda", generator=g)
    dst = torch.zeros(96 << 20, dtype=torch.uint8, pin_memory=True)
    sb = SaveBackEngine(torch.cuda.current_device())
    sb.submit(_items([(dst, src)]), _stream())
    sb.close()
    assert torch.equal(dst, src.cpu())


@pytest.mark.parametrize("mode", ["sdma", "stream"])
def test_engine_save_backs_then_load_waits_for_them(mode):
    """``d2h_async`` / ``d2h_into`` on either engine, then a load whose pinned pieces are the
    save-back's outputs, submitted before the save-back finished: the load waits for it (in the
    loader's worker for a ticket, on the device for an event)."""
    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool, save_back=mode)
    kind = SaveBackTicket if mode == "sdma" else NativeEvent
    g = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randint(0, 256, (3 << 19,), dtype=torch.uint8, device="cuda", generator=g)
    b = torch.randint(0, 256, (5000,), dtype=torch.uint8, device="cuda", generator=g)
    (ha, hb), done = eng.d2h_async([a, b])
    assert isinstance(done, kind)
    block = torch.randint(0, 256, ((24 << 20) + 6,), dtype=torch.uint8, device="cuda", generator=g)
    home = torch.zeros(block.numel() + 10, dtype=torch.uint8, pin_memory=True)
    done2 = eng.d2h_into(block, home[:block.numel()])
    assert isinstance(done2, kind)
    pageable = torch.randint(0, 256, ((5 << 19) + 7,), dtype=torch.uint8)
    layout = [(0, home[:block.numel()]), (block.numel(), ha), (block.numel() + ha.numel(), pageable),
              (block.numel() + ha.numel() + pageable.numel(), hb)]
    total = sum(t.numel() for _o, t in layout)
    dst = torch.zeros(total, dtype=torch.uint8, device="cuda")
    h = eng.submit_block_load("mixed", BlockSource(layout, total), dst, wait_event=done2)
    eng.wait(h)
    assert torch.equal(dst.cpu(), torch.cat([block.cpu(), a.cpu(), pageable, b.cpu()]))
    assert eng.bytes_d2h == a.numel() + b.numel() + block.numel()
    eng.shutdown()
    pool.shutdown()


def test_trace_reports_copy_engine_spans():
    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool, save_back="sdma")
    g = torch.Generator(device="cuda").manual_seed(5)
    srcs = [torch.randint(0, 256, (64 << 20,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(3)]
    homes = [torch.zeros(64 << 20, dtype=torch.uint8, pin_memory=True) for _ in range(3)]
    eng.start_trace()
    for s, h in zip(srcs, homes):
        eng.d2h_into(s, h)
    tr = eng.stop_trace()
    spans = [(n, t0, t1, fence, sub) for n, t0, t1, kind, fence, sub in tr["d2h"] if kind == "block"]
    assert len(spans) == 3
    for n, t0, t1, fence, sub in spans:
        assert n == 64 << 20
        assert -1.0 < t0 < t1 < 10_000.0
        assert n / ((t1 - t0) * 1e-3) < 100e9  # no faster than a PCIe link can go
        # the copy starts after the device passed its fence (the copy engine's clock and the HIP
        # timeline are aligned to within a millisecond), which it reaches after the host submits
        assert -1.0 < fence <= t0 + 1.0 and sub >= 0.0
    for s, h in zip(srcs, homes):
        assert torch.equal(h, s.cpu())
    eng.shutdown()
    pool.shutdown()


@pytest.mark.parametrize("mode", ["sdma", "stream"])
def test_released_memory_is_counted_until_reaped_and_bounded(mode):
    """``release_with_copy`` counts a buffer as released while its save-back holds it;
    ``wait_releasing`` waits for the oldest save-backs until at most the given bytes remain."""
    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool, save_back=mode)
    g = torch.Generator(device="cuda").manual_seed(6)
    n = 32 << 20
    srcs = [torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(4)]
    homes = [torch.zeros(n, dtype=torch.uint8, pin_memory=True) for _ in range(4)]
    done = [eng.d2h_into(s, h) for s, h in zip(srcs, homes)]
    assert all(eng.release_with_copy(d, n) for d in done)
    assert not eng.release_with_copy(NativeEvent(), n)  # not a save-back in flight
    assert eng.releasing_bytes() <= 4 * n
    eng.wait_releasing(n)
    assert eng.releasing_bytes() <= n
    for d in done[:3]:
        assert d.query()
    eng.wait_releasing(0)
    assert eng.releasing_bytes() == 0
    for s, h in zip(srcs, homes):
        assert torch.equal(h, s.cpu())
    eng.shutdown()
    pool.shutdown()


def test_release_of_earlier_tickets_while_a_later_one_is_waited_for():
    """A waiter on a later ticket holds every earlier job it waits for; releasing those tickets
    from another thread meanwhile drops only the engine's reference (the signals stay valid
    until the waiter is done). Also: a ticket with no copies completes at once and may be
    dropped before anything else happens."""
    import threading

    g = torch.Generator(device="cuda").manual_seed(7)
    n = 24 << 20
    srcs = [torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(8)]
    dsts = [torch.zeros(n, dtype=torch.uint8, pin_memory=True) for _ in range(8)]
    sb = SaveBackEngine(torch.cuda.current_device())
    lib, h = _native.lib(), sb.handle
    for rep in range(4):
        a = torch.randn(2048, 2048, device="cuda")
        for _ in range(8):  # the copies wait behind queued compute, so the waiter really waits
            a = a @ a * 1e-3
        tickets = [sb.submit(_items([(d, s)]), _stream()) for d, s in zip(dsts, srcs)]
        result = {}

        def waiter():
            result["st"] = lib.sh_saveback_wait(h, ctypes.c_uint64(tickets[-1].ticket))

        th = threading.Thread(target=waiter)
        th.start()
        for t in tickets[:-1]:
            assert lib.sh_saveback_release(h, ctypes.c_uint64(t.ticket)) == _native.SH_OK
        th.join(timeout=60)
        assert not th.is_alive(), rep
        assert result["st"] == _native.SH_OK, rep
        for d, s in zip(dsts, srcs):
            assert torch.equal(d, s.cpu()), rep
        del tickets
    sb.close()

    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool, save_back="sdma")
    empty_src = torch.empty(0, dtype=torch.uint8, device="cuda")
    empty_dst = torch.empty(0, dtype=torch.uint8, pin_memory=True)
    done = eng.d2h_into(empty_src, empty_dst)
    assert isinstance(done, SaveBackTicket) and done.query()
    del done  # released at once: no copy, no fence for the worker to wait on
    later = eng.d2h_into(srcs[0], dsts[1])
    later.synchronize()
    assert torch.equal(dsts[1], srcs[0].cpu())
    eng.drain()
    eng.shutdown()
    pool.shutdown()


def test_submit_after_waits_for_its_events_not_for_the_stream():
    """``submit_after`` copies once its events have completed, while the stream they were recorded
    on is still busy; with no events it copies at once. Both complete in submission order."""
    import time

    from tests.test_streaming_gpu import _sleep_cycles_for

    sb = SaveBackEngine(torch.cuda.current_device())
    g = torch.Generator(device="cuda").manual_seed(9)
    srcs = [torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g) for n in (16 << 20, 4097)]
    dsts = [torch.zeros(s.numel(), dtype=torch.uint8, pin_memory=True) for s in srcs]
    ready = NativeEvent()
    ready.record(_stream())  # the sources are final here
    spin = _sleep_cycles_for(400.0)
    torch.cuda._sleep(spin)
    t0 = time.perf_counter()
    first = sb.submit_after(_items([(dsts[0], srcs[0])]), [ready])
    second = sb.submit_after(_items([(dsts[1], srcs[1])]), [])
    second.synchronize()  # covers the first ticket too
    took = time.perf_counter() - t0
    assert first.query() and took < 0.2, f"{took * 1e3:.0f} ms"
    for d, s in zip(dsts, srcs):
        assert torch.equal(d, s.cpu())
    with pytest.raises(ValueError, match="event 0 is NULL"):
        import types

        sb.submit_after(_items([(dsts[1], srcs[1])]), [types.SimpleNamespace(handle=ctypes.c_void_p())])
    torch.cuda.synchronize()
    sb.close()


@pytest.mark.parametrize("n,chunk", [((6 << 20) + 7, 1 << 20), (3 * 4096, 4096), (4096 * 40 + 16, 4096)])
def test_submit_chunks_copies_the_changed_chunks(n, chunk):
    """The chunk form of a save-back: the host buffer holds what the digests describe, the device
    buffer then changes in some chunks (the first, the last partial one, two adjacent ones, one
    alone); after the ticket the host buffer equals the device buffer, only the changed chunks were
    copied (adjacent ones as one run), and with no change nothing is copied."""
    lib = _native.lib()
    g = torch.Generator(device="cuda").manual_seed(n)
    dev = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    n_chunks = -(-n // chunk)
    host = torch.empty(n + 64, dtype=torch.uint8, pin_memory=True)
    host[:n].copy_(dev.cpu())
    host[n:] = 0xEE
    dig = torch.zeros(2 * n_chunks, dtype=torch.int64, device="cuda")
    assert lib.sh_block_digest(dev.data_ptr(), n, chunk, dig.data_ptr(), _stream()) == _native.SH_OK
    flags = torch.zeros(n_chunks, dtype=torch.uint8, pin_memory=True)
    eng = AsyncTransferEngine(PinnedPool(total_mb=4, slab_mb=1, alignment=512), save_back="sdma")
    sb = eng._saveback_engine()
    unpack = eng._loader_unpack_stream()

    region = [(host.data_ptr(), dev.data_ptr(), n)]
    t = sb.submit_chunks(region, chunk, dig.data_ptr(), flags.data_ptr(), unpack, None, _stream())
    assert t.copied_bytes() == 0
    hit = sorted({0, n_chunks - 1, 1, 2, n_chunks // 2 + 1} & set(range(n_chunks)))
    for c in hit:
        dev[min(c * chunk + 3, n - 1)] += 1
    t = sb.submit_chunks(region, chunk, dig.data_ptr(), flags.data_ptr(), unpack, None, _stream())
    copied = t.copied_bytes()
    assert copied == sum(min(chunk, n - c * chunk) for c in hit)
    assert torch.equal(host[:n], dev.cpu()) and (host[n:] == 0xEE).all()
    np.testing.assert_array_equal(np.flatnonzero(flags.numpy()), hit)
    # without digests: every chunk, in one run
    dev.add_(3)
    t = sb.submit_chunks(region, chunk, 0, 0, unpack, None, _stream())
    assert t.copied_bytes() == n and torch.equal(host[:n], dev.cpu())
    eng.shutdown()


def test_d2h_changed_waits_for_its_events_and_counts_copied_bytes():
    """``AsyncTransferEngine.d2h_changed`` after caller events: the comparison runs once the events
    have passed (a write queued before them is seen), and ``bytes_d2h`` counts the copied chunks
    when the ticket is reaped."""
    chunk = 1 << 20
    n = 8 * chunk
    eng = AsyncTransferEngine(PinnedPool(total_mb=4, slab_mb=1, alignment=512), save_back="sdma")
    dev = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    host = dev.cpu().pin_memory()
    dig = torch.zeros(16, dtype=torch.int64, device="cuda")
    assert _native.lib().sh_block_digest(dev.data_ptr(), n, chunk, dig.data_ptr(), _stream()) == _native.SH_OK
    flags = torch.zeros(8, dtype=torch.uint8, pin_memory=True)
    torch.cuda._sleep(50_000_000)
    dev[5 * chunk + 17] += 1  # queued behind the spin
    ev = eng.record_event()
    before = eng.bytes_d2h
    t = eng.d2h_changed(dev, host, chunk, dig, flags, after=[ev])
    t.synchronize()
    eng.reap()
    assert torch.equal(host, dev.cpu())
    assert np.flatnonzero(flags.numpy()).tolist() == [5]
    assert eng.bytes_d2h - before == chunk and eng.bytes_d2h_requested == n
    eng.shutdown()


def test_whole_queue_fence_sees_writes_through_param_data():
    """``save_back_fence="whole_queue"``: a write through ``param.data`` (which leaves the
    parameter's version counter alone) queued after the block's last use, behind a long run of
    kernels, and then the block's training eviction inside the step: the host copy holds the
    write, as the reference's synchronous ``param.data.to("cpu")`` (scheduler.py:1216-1226) sees
    it. The default fence takes the block's last use instead, which does not order the copy after
    such a write (the case the switch exists for)."""
    import stagehand_amd as stagehand
    from stagehand_amd.config import StagehandConfig
    from tests.streaming_models import TinyStack, init_

    for fence in ("whole_queue", "last_use"):
        model = init_(TinyStack(n=3, hidden=256, mlp=4)).to(torch.bfloat16)
        cfg = StagehandConfig(pinned_pool_mb=64, pinned_slab_mb=4, vram_high_watermark_mb=200000,
                              vram_low_watermark_mb=100000, prefetch_window_blocks=1, telemetry_enabled=False,
                              nan_inf_check=False, strict_bf16=False, save_back_fence=fence,
                              save_back_changed_chunks=False)
        rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                        inference_mode=False)
        sched = rt._scheduler
        x = torch.randn(4, 256).to(torch.bfloat16).cuda()
        rt.begin_step(0)
        with rt.managed_forward():
            model(x).float().sum().backward()
        w = model.blocks[0].fc1.weight
        assert w.is_cuda
        a = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
        for _ in range(30):  # keeps the device busy well past the eviction's submit
            a = torch.tanh(a @ a)
        v0 = w._version
        w.data.fill_(0.25)  # through .data: the version counter does not move
        assert w._version == v0
        sched._evict_block("blocks.0", save_back=True)
        host = model.blocks[0].fc1.weight
        assert not host.is_cuda
        if fence == "whole_queue":
            assert bool((host.float() == 0.25).all()), "the save-back ran before the write through param.data"
            assert sched.fence_kinds["whole_queue_configured"] >= 1
        else:
            assert sched.fence_kinds["whole_queue_configured"] == 0
        rt.end_step()
        torch.cuda.synchronize()
        rt.shutdown()
