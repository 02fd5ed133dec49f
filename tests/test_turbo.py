"""Turbo window engine (stagehand_amd.turbo over sh_turbo_* in the C ABI).

CPU tests pin the API surface and error mapping of the reference's pyo3 class
(turbo_src/lib.rs:14-126: ValueError for a bad direction, RuntimeError for
everything else, None for a block without a slot). GPU tests check that every
byte a block lands in its slot equals the staged bytes, in the reference's
per-parameter slot mode and in the contiguous mode, the location state machine
(engine.rs:384-393), the forward/backward window policy (engine.rs:304-341),
write-back on and off, and that a model streamed through the conductor gives
bit-identical outputs to the same model resident on the device.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from stagehand_amd.turbo import TransferEngine, TurboConductor

from tests.streaming_models import TinyStack, init_


def test_api_without_device():
    e = TransferEngine()
    assert e.register_block([100, 0, 300]) == 0
    assert e.register_block([10]) == 1
    assert (e.num_blocks(), e.num_gpu_slots(), e.num_free_slots()) == (2, 0, 0)
    assert e.block_location(0) == "cpu" and e.block_slot(0) is None and e.block_slot(7) is None
    assert [e.param_offset(0, p) for p in range(3)] == [0, 256, 256]  # 256-byte aligned offsets
    assert e.slot_bytes() == 768
    with pytest.raises(ValueError, match="forward"):
        e.step(0, "sideways")
    with pytest.raises(RuntimeError, match="not initialized"):
        e.step(0, "forward")
    with pytest.raises(RuntimeError):
        e.block_location(5)
    with pytest.raises(RuntimeError):
        e.gpu_ptr(0, 0)
    with pytest.raises(RuntimeError):
        e.cpu_ptr(0, 9)
    e.close()


def test_conductor_needs_matching_blocks():
    with pytest.raises(ValueError, match="No blocks matched"):
        TurboConductor(torch.nn.Linear(4, 4), block_pattern=r"^nothing$")


def test_conductor_rejects_a_window_below_three():
    with pytest.raises(ValueError, match="window must be at least 3"):
        TurboConductor(torch.nn.Sequential(torch.nn.Linear(4, 4)), block_pattern=r"^0$", window=2)
    with pytest.raises(ValueError, match="save_back"):
        TurboConductor(torch.nn.Sequential(torch.nn.Linear(4, 4)), block_pattern=r"^0$", save_back="dma")


# ── GPU ─────────────────────────────────────────────────────────────────


def _blocks(seed: int, n: int, sizes_fn):
    g = torch.Generator().manual_seed(seed)
    data = []
    for i in range(n):
        data.append([torch.randint(0, 256, (s,), dtype=torch.uint8, generator=g) for s in sizes_fn(i)])
    return data


@pytest.mark.gpu
@pytest.mark.parametrize("save_back", ["sdma", "stream"])
def test_per_param_slots_land_every_byte(save_back):
    """Reference usage: slot pointers per parameter position, sized to the largest block."""
    sizes = lambda i: [4096 + 512 * (i % 3), 1000 + i, 0, 77 * (i + 1)]  # ragged, one empty param
    data = _blocks(1, 7, sizes)
    e = TransferEngine()
    for d in data:
        e.register_block([t.numel() for t in d])
    e.set_save_back(save_back)
    e.initialize(torch.cuda.current_device(), 3)
    assert (e.num_gpu_slots(), e.num_free_slots()) == (3, 3)
    for i, d in enumerate(data):
        e.stage_block(i, [t.data_ptr() for t in d])
    cap = [max(d[p].numel() for d in data) for p in range(4)]
    slots = [[torch.empty(max(c, 1), dtype=torch.uint8, device="cuda") for c in cap] for _ in range(3)]
    for s, ts in enumerate(slots):
        e.set_slot_gpu_ptrs(s, [t.data_ptr() for t in ts])
    for direction, order in (("forward", range(7)), ("backward", reversed(range(7)))):
        for i in order:
            e.step(i, direction)
            s = e.block_slot(i)
            assert s is not None and e.block_location(i) == "gpu"
            torch.cuda.current_stream().synchronize()
            for p, t in enumerate(data[i]):
                if t.numel():
                    assert e.gpu_ptr(i, p) == slots[s][p].data_ptr()
                    assert torch.equal(slots[s][p][:t.numel()].cpu(), t)
            nxt = i + 1 if direction == "forward" else i - 1
            if 0 <= nxt < 7:
                assert e.block_location(nxt) in ("h2d", "gpu")
    e.drain()
    assert all(e.block_location(i) in ("cpu", "gpu", "h2d") for i in range(7))
    e.close()


@pytest.mark.gpu
@pytest.mark.parametrize("save_back", ["sdma", "stream"])
def test_contiguous_slots_one_copy_per_block_and_writeback(save_back):
    sizes = lambda i: [3000 + i, 5000, 123]
    data = _blocks(2, 5, sizes)
    e = TransferEngine()
    for d in data:
        e.register_block([t.numel() for t in d])
    e.set_save_back(save_back)
    e.initialize(torch.cuda.current_device(), 3)
    for i, d in enumerate(data):
        e.stage_block(i, [t.data_ptr() for t in d])
    nb = e.slot_bytes()
    slots = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(3)]
    for s, t in enumerate(slots):
        e.set_slot_buffer(s, t.data_ptr(), nb)
    e.set_writeback(1, False)  # frozen
    for i in range(5):
        e.step(i, "forward")
        torch.cuda.current_stream().synchronize()
        base = slots[e.block_slot(i)]
        for p, t in enumerate(data[i]):
            off = e.param_offset(i, p)
            assert e.gpu_ptr(i, p) == base.data_ptr() + off
            assert torch.equal(base[off:off + t.numel()].cpu(), t)
        # modify block i on the device, as an optimizer step would
        base[e.param_offset(i, 0)] += 1
    e.drain()
    h2d, d2h = e.bytes_moved()
    ext = [e.param_offset(i, 2) + 256 for i in range(5)]  # last param (123 B) rounds up to 256
    assert h2d == sum(ext)  # one contiguous copy of each block, each block once
    assert d2h == sum(ext[i] for i in (0, 2, 3))  # blocks 0, 2 and 3 were evicted; block 1 has write-back off
    for i, want_bump in ((0, True), (1, False), (2, True), (3, True)):
        assert e.block_location(i) == "cpu"
        p0 = data[i][0]
        buf = (ctypes.c_uint8 * p0.numel()).from_address(e.cpu_ptr(i, 0))
        got = torch.frombuffer(buf, dtype=torch.uint8)
        want = p0.clone()
        if want_bump:
            want[0] += 1
        assert torch.equal(got, want), i
    e.close()


@pytest.mark.gpu
@pytest.mark.parametrize("save_back", ["sdma", "stream"])
def test_written_back_blocks_reload_with_their_updates(save_back):
    """Forward: every block is changed on the device right after its step, with kernels still
    queued when the next step evicts it. Backward: each block reloads from its written-back host
    region (through slots that the write-backs were still reading) and carries the change."""
    sizes = lambda i: [(1 << 20) + 4096 * i, 3 << 18, 999]
    data = _blocks(3, 6, sizes)
    e = TransferEngine()
    for d in data:
        e.register_block([t.numel() for t in d])
    e.set_save_back(save_back)
    e.initialize(torch.cuda.current_device(), 3)
    for i, d in enumerate(data):
        e.stage_block(i, [t.data_ptr() for t in d])
    nb = e.slot_bytes()
    slots = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(3)]
    for s, t in enumerate(slots):
        e.set_slot_buffer(s, t.data_ptr(), nb)
    a = torch.randn(2048, 2048, device="cuda")
    for rnd in range(2):
        for direction, order in (("forward", range(6)), ("backward", reversed(range(6)))):
            for i in order:
                e.step(i, direction)
                base = slots[e.block_slot(i)]
                for _ in range(3):  # keep the compute stream busy past the next eviction
                    a = (a @ a) * 1e-3
                for p in range(3):
                    off = e.param_offset(i, p)
                    view = base[off:off + data[i][p].numel()]
                    view.add_(1)
                    data[i][p] += 1
        torch.cuda.synchronize()
    e.drain()
    for i in range(6):
        e.step(i, "forward")
        torch.cuda.current_stream().synchronize()
        base = slots[e.block_slot(i)]
        for p, want in enumerate(data[i]):
            off = e.param_offset(i, p)
            assert torch.equal(base[off:off + want.numel()].cpu(), want), (i, p)
    e.drain()
    e.close()


@pytest.mark.gpu
def test_no_free_slot_is_runtime_error():
    e = TransferEngine()
    for _ in range(2):
        e.register_block([1024])
    e.initialize(torch.cuda.current_device(), 1)
    buf = torch.empty(1024, dtype=torch.uint8, device="cuda")
    e.set_slot_buffer(0, buf.data_ptr(), 1024)
    src = torch.zeros(1024, dtype=torch.uint8)
    e.stage_block(0, [src.data_ptr()])
    e.stage_block(1, [src.data_ptr()])
    e.step(0, "forward")  # the lookahead prefetch of block 1 finds no slot: not an error
    assert e.block_location(1) == "cpu"
    with pytest.raises(RuntimeError, match="No free GPU slots"):
        e.step(1, "forward")
    e.evict_sync(0)
    assert e.block_location(0) == "cpu" and e.num_free_slots() == 1
    e.step(1, "forward")
    assert e.block_location(1) == "gpu"
    e.drain()
    e.close()


@pytest.mark.gpu
def test_conductor_forward_matches_resident_model():
    model = init_(TinyStack(n=6, hidden=64, mlp=4), seed=3).to(torch.bfloat16)
    model.requires_grad_(False)
    ref = init_(TinyStack(n=6, hidden=64, mlp=4), seed=3).to(device="cuda", dtype=torch.bfloat16)
    x = torch.randn(8, 64, generator=torch.Generator().manual_seed(4)).to("cuda", torch.bfloat16)
    cond = TurboConductor(model, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16)
    cond.prepare()
    # non-block parameters stay where they are; here every parameter is in a block
    handles = cond.install_hooks()
    with torch.no_grad():
        outs = [model(x) for _ in range(3)]
        want = ref(x)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))
    h2d, d2h = cond.engine.bytes_moved()
    assert d2h == 0  # frozen: no write-back
    # the last block keeps its slot between steps (engine.rs:304-341 evicts only the
    # previous block), so after the first pass each step loads 5 of the 6 blocks, one
    # copy of the block's aligned extent each
    assert h2d == (6 + 5 + 5) * cond.engine.slot_bytes()
    assert cond.engine.slot_bytes() >= sum(p.numel() * 2 for p in ref.blocks[0].parameters())
    for h in handles:
        h.remove()
    cond.shutdown()
    for p, q in zip(model.parameters(), ref.parameters()):
        assert torch.equal(p.view(torch.int16), q.cpu().view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("window,chunk", [(3, 0), (4, 0), (3, 1 << 20)])
def test_conductor_with_writeback_and_other_windows_matches_resident_model(window, chunk):
    """Write-back of every block (the reference's engine) through 3 or 4 slots: outputs match the
    resident model and the host copies are unchanged after three passes. Write-backs of every byte
    move bytes back; write-backs of changed chunks move none (inference writes no weight)."""
    model = init_(TinyStack(n=6, hidden=64, mlp=4), seed=7).to(torch.bfloat16)
    model.requires_grad_(False)
    ref = init_(TinyStack(n=6, hidden=64, mlp=4), seed=7).to(device="cuda", dtype=torch.bfloat16)
    x = torch.randn(8, 64, generator=torch.Generator().manual_seed(8)).to("cuda", torch.bfloat16)
    cond = TurboConductor(model, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16, writeback="always",
                          window=window, writeback_chunk_bytes=chunk)
    cond.prepare()
    assert cond.engine.num_gpu_slots() == window
    handles = cond.install_hooks()
    with torch.no_grad():
        outs = [model(x) for _ in range(3)]
        want = ref(x)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))
    h2d, d2h = cond.engine.bytes_moved()
    assert d2h > 0 if chunk == 0 else d2h == 0
    for h in handles:
        h.remove()
    cond.shutdown()
    for p, q in zip(model.parameters(), ref.parameters()):
        assert torch.equal(p.view(torch.int16), q.cpu().view(torch.int16))


@pytest.mark.gpu
def test_trace_records_every_write_back_and_host_wait():
    """A traced pass with write-back of every byte of every block in the reference's per-parameter
    layout: one
    write-back span per evicted block with the block's bytes, timed by the copy engine after that
    block's compute began, and host waits that end after they start."""
    model = init_(TinyStack(n=6, hidden=64, mlp=4), seed=9).to(torch.bfloat16)
    model.requires_grad_(False)
    x = torch.randn(8, 64, generator=torch.Generator().manual_seed(10)).to("cuda", torch.bfloat16)
    cond = TurboConductor(model, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16, writeback="always",
                          contiguous_slots=False, writeback_chunk_bytes=0)
    cond.prepare()
    handles = cond.install_hooks()
    with torch.no_grad():
        model(x)
        torch.cuda.synchronize()
        cond.start_trace()
        model(x)
        trace = cond.stop_trace()
    # step(i) evicts block i-1: blocks 0-4 are written back during the pass, block 5 keeps its slot
    assert trace["d2h_untimed"] == 0
    assert len(trace["d2h"]) == 5
    block_bytes = sum(p.numel() * 2 for p in model.blocks[0].parameters())
    starts = {name: s for name, s, _e in trace["compute"]}
    for k, (nbytes, t0, t1, kind) in enumerate(trace["d2h"]):
        assert kind == "writeback" and nbytes == block_bytes
        assert 0 < t0 <= t1
        # the copy engine's clock and the HIP timeline are aligned to within a millisecond here
        assert t0 >= starts[f"blocks.{k}"] - 1.0
    for kind, t0, t1 in trace["host_waits"]:
        assert kind == "slot_reuse" and t0 <= t1
    for h in handles:
        h.remove()
    cond.shutdown()


def _sleep_cycles_for(ms: float) -> int:
    """Cycles of torch.cuda._sleep (a bounded spin kernel) that keep the current stream busy for
    about ``ms`` milliseconds on this device."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    probe = 1_000_000
    torch.cuda._sleep(probe)  # first launch loads the kernel
    start.record()
    torch.cuda._sleep(probe)
    end.record()
    end.synchronize()
    per_ms = probe / max(start.elapsed_time(end), 1e-3)
    return int(min(per_ms * ms, 4_000_000_000))


@pytest.mark.gpu
def test_lookahead_behind_a_write_back_is_issued_by_the_next_step():
    """When every free slot is still the source of a write-back waiting for queued compute, step()
    does not block the host on it: the lookahead block is marked h2d and the next step issues its
    copy after the write-back. Every block still lands byte-exact and the write-back carries the
    change made on the device."""
    import time

    sizes = lambda i: [(1 << 20) + 512 * i, 4096]
    data = _blocks(5, 4, sizes)
    e = TransferEngine()
    for d in data:
        e.register_block([t.numel() for t in d])
    e.set_save_back("sdma")
    e.initialize(torch.cuda.current_device(), 3)
    for i, d in enumerate(data):
        e.stage_block(i, [t.data_ptr() for t in d])
    nb = e.slot_bytes()
    slots = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(3)]
    for s, t in enumerate(slots):
        e.set_slot_buffer(s, t.data_ptr(), nb)
    spin = _sleep_cycles_for(300.0)
    e.set_timing(True)
    e.step(0, "forward")            # block 0 into slot 0, lookahead 1 into slot 1
    torch.cuda._sleep(spin)         # block 0's compute: both write-backs below wait for it
    e.step(1, "forward")            # evicts 0; lookahead 2 takes the unused slot 2
    base = slots[e.block_slot(1)]
    base[e.param_offset(1, 0)] += 1
    data[1][0][0] += 1
    t0 = time.perf_counter()
    e.step(2, "forward")            # evicts 1; lookahead 3 can only reuse slot 0 or 1
    host_s = time.perf_counter() - t0
    assert host_s < 0.15, f"step() waited {host_s * 1e3:.0f} ms for a write-back"
    assert e.block_location(3) == "h2d"
    e.step(3, "forward")            # issues block 3's copy once block 0's write-back is done
    torch.cuda.synchronize()
    base = slots[e.block_slot(3)]
    for p, want in enumerate(data[3]):
        off = e.param_offset(3, p)
        assert torch.equal(base[off:off + want.numel()].cpu(), want), p
    spans = e.trace_spans()
    waits = spans[spans["kind"] == 1]
    assert len(waits) >= 1 and all(int(w["block"]) == 3 for w in waits)
    e.set_timing(False)
    e.drain()
    for i in range(3):
        assert e.block_location(i) == "cpu"
        for p, want in enumerate(data[i]):
            buf = (ctypes.c_uint8 * want.numel()).from_address(e.cpu_ptr(i, p))
            assert torch.equal(torch.frombuffer(buf, dtype=torch.uint8), want), (i, p)
    e.close()


@pytest.mark.gpu
@pytest.mark.parametrize("contiguous", [True, False])
def test_writebacks_copy_the_changed_chunks(contiguous):
    """Write-backs of changed chunks: after each H2D the engine takes chunk digests of the slot, and
    a write-back copies back only the chunks written on the device since. Two bytes change in each
    of blocks 0, 2 and 4 (one in the first parameter past its first chunk, one in the small last
    parameter); blocks 1 and 3 are only read. The host regions then equal the slots' bytes, exactly
    the changed chunks were copied (per parameter in the reference's layout of one slot tensor per
    parameter, over the whole block in a contiguous slot), and reloading carries the changes."""
    chunk = 1 << 16
    sizes = lambda i: [(3 << 20) + 100, 2 << 20, 5000]
    data = _blocks(9, 5, sizes)
    e = TransferEngine()
    for d in data:
        e.register_block([t.numel() for t in d])
    e.set_save_back("sdma")
    e.set_writeback_chunks(chunk)
    e.initialize(torch.cuda.current_device(), 3)
    for i, d in enumerate(data):
        e.stage_block(i, [t.data_ptr() for t in d])
    if contiguous:
        nb = e.slot_bytes()
        slots = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(3)]
        for s, t in enumerate(slots):
            e.set_slot_buffer(s, t.data_ptr(), nb)
    else:
        cap = [t.numel() for t in data[0]]
        slots = [[torch.empty(c, dtype=torch.uint8, device="cuda") for c in cap] for _ in range(3)]
        for s, ts in enumerate(slots):
            e.set_slot_gpu_ptrs(s, [t.data_ptr() for t in ts])

    def param_view(i, p):
        s = e.block_slot(i)
        if contiguous:
            off = e.param_offset(i, p)
            return slots[s][off:off + data[i][p].numel()]
        return slots[s][p][:data[i][p].numel()]

    changed = (0, 2, 4)
    for i in range(5):
        e.step(i, "forward")
        if i in changed:
            param_view(i, 0)[70000] += 1
            param_view(i, 2)[10] += 1
            data[i][0][70000] += 1
            data[i][2][10] += 1
    e.drain()
    _h2d, d2h = e.bytes_moved()
    if contiguous:
        ext = e.param_offset(0, 2) + 5120  # 5000 B rounded up to 256
        dirty = {70000 // chunk, (e.param_offset(0, 2) + 10) // chunk}
        per_block = sum(min(chunk, ext - c * chunk) for c in dirty)
    else:
        per_block = chunk + 5000  # one chunk of parameter 0, all of parameter 2
    # blocks 0-3 were evicted by the forward steps; block 4 keeps its slot
    assert d2h == 2 * per_block
    for i in range(4):
        assert e.block_location(i) == "cpu"
        for p, want in enumerate(data[i]):
            buf = (ctypes.c_uint8 * want.numel()).from_address(e.cpu_ptr(i, p))
            assert torch.equal(torch.frombuffer(buf, dtype=torch.uint8), want), (i, p)
    for i in reversed(range(5)):
        e.step(i, "backward")
        torch.cuda.current_stream().synchronize()
        for p, want in enumerate(data[i]):
            assert torch.equal(param_view(i, p).cpu(), want), (i, p)
    e.drain()
    e.close()
