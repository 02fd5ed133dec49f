"""The block loader's post-copy work (a plan's unpack, chunk digests) through every way a load is
consumed.

The loader queues that work on the first call that needs it: ``sh_loader_stream_wait`` on the
waiting stream, ``sh_loader_query`` / ``sync`` / ``release`` on the loader's unpack stream once the
copy has landed. Each path must leave the same bytes: the int8 rows dequantised and the fp32
values cast as the oracle says (oracle/squareq.py: src/stagehand/scheduler.py:285-300, :181),
bit for bit, and the digests equal to their restated definition (tests/test_digest.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import squareq as oq
from stagehand_amd.pool import PinnedPool
from stagehand_amd.transfer import AsyncTransferEngine, BlockSource
from stagehand_amd.unpack import KIND_F32_BF16, KIND_I8_ROWSCALE_BF16, UnpackPlan, make_descs
from test_digest import digest_np

pytestmark = pytest.mark.gpu

ROWS, COLS, NF = 96, 3072, 70_001  # 576 KiB of bf16 rows + 137 KiB of cast values: several chunks
CHUNK = 64 << 10


def _block(seed: int):
    """Source bytes (int8 rows, their fp32 scales, fp32 values), the plan, and the expected bf16."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-128, 128, size=(ROWS, COLS), dtype=np.int8)
    s = (rng.standard_normal(ROWS) * 1e-2).astype(np.float32)
    f = (rng.standard_normal(NF) * 3).astype(np.float32)
    f[:4] = [np.inf, -np.inf, np.nan, 1e-40]
    q_off, s_off = 0, ROWS * COLS
    f_off = s_off + 4 * ROWS
    src = np.zeros(f_off + 4 * NF, dtype=np.uint8)
    src[q_off:s_off] = q.view(np.uint8).reshape(-1)
    src[s_off:f_off] = s.view(np.uint8)
    src[f_off:] = f.view(np.uint8)
    plan = UnpackPlan(make_descs([(KIND_I8_ROWSCALE_BF16, q_off, 0, ROWS, COLS, 0, 0),
                                  (KIND_F32_BF16, f_off, 2 * ROWS * COLS, 1, NF, 0, 0)]))
    want = np.concatenate([oq.dequant_rows(q, s, None, ROWS, COLS).reshape(-1), oq.cast_f32_bf16(f)])
    return src, s_off, plan, want


@pytest.mark.parametrize("how", ["stream_wait", "query", "sync", "release"])
def test_post_copy_work_runs_on_every_consumption_path(how):
    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool)
    try:
        for seed in range(3):  # three loads in a row: events and tickets are reused
            src, s_off, plan, want = _block(seed)
            dst_bytes = 2 * want.size
            dst = torch.full((dst_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
            n_chunks = -(-dst_bytes // CHUNK)
            dig = torch.zeros(2 * n_chunks, dtype=torch.int64, device="cuda")
            source = BlockSource([(0, torch.from_numpy(src))], src.size, plan=plan, scale_off=s_off, n_scale=ROWS)
            h = eng.submit_block_load(f"b{seed}", source, dst, digest=(dig, dst_bytes, CHUNK))
            if how == "stream_wait":
                side = torch.cuda.Stream()
                with torch.cuda.stream(side):
                    eng.wait_device(h)
                    got = dst.clone()  # ordered after the unpack on this stream
                side.synchronize()
                got_dig = dig.clone()
                eng.wait(h)
            elif how == "query":
                while not eng.poll(h):
                    pass
                got, got_dig = dst.clone(), dig.clone()
            elif how == "sync":
                eng.wait(h)
                got, got_dig = dst.clone(), dig.clone()
            else:
                eng._complete_handle(h)  # released with no wait before it
                got, got_dig = dst.clone(), dig.clone()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), want)
            np.testing.assert_array_equal(got_dig.cpu().numpy().view(np.uint64),
                                          digest_np(want.view(np.uint8), CHUNK).reshape(-1))
    finally:
        eng.shutdown()
        pool.shutdown()


def test_inflight_bound_counts_copies_not_post_copy_work():
    """The in-flight bound (the reference's max_inflight, src/stagehand/transfer.py:258-276) limits
    copies: a load whose unpack waits on a busy stream, behind work the host queued ahead, holds
    no slot once its copy has landed, and the next submit does not wait for that stream.

    Everything that may synchronise the device (plan creation copies its tables with hipMemcpy;
    freeing device memory, as the garbage collection of an earlier test's plan would, waits for
    the whole device) happens before the busy stream's spin is queued, with the collector paused."""
    import gc

    from test_streaming_gpu import _sleep_cycles_for

    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool, max_inflight=1)
    busy = torch.cuda.Stream()
    cycles = _sleep_cycles_for(400.0)
    src, s_off, plan, want = _block(7)
    src2, s_off2, plan2, want2 = _block(8)
    dst = torch.empty(2 * want.size, dtype=torch.uint8, device="cuda")
    dst2 = torch.empty(2 * want2.size, dtype=torch.uint8, device="cuda")
    # two staging buffers of the loads' size in the allocator's cache, so the submits allocate nothing
    warm = [torch.empty(max(src.size, src2.size), dtype=torch.uint8, device="cuda") for _ in range(2)]
    del warm
    source = BlockSource([(0, torch.from_numpy(src))], src.size, plan=plan, scale_off=s_off, n_scale=ROWS)
    source2 = BlockSource([(0, torch.from_numpy(src2))], src2.size, plan=plan2, scale_off=s_off2, n_scale=ROWS)
    # one load through the same path first: the loader, its streams and the kernels are set up
    hw = eng.submit_block_load("warm-up", source, dst)
    eng.wait_device(hw)
    eng.wait(hw)
    gc.collect()
    torch.cuda.synchronize()
    gc.disable()
    try:
        h1 = eng.submit_block_load("first", source, dst)
        with torch.cuda.stream(busy):
            torch.cuda._sleep(cycles)  # about 400 ms of device work queued ahead
            eng.wait_device(h1)        # the unpack goes behind it
        while eng._copy_outstanding(h1):
            pass
        eng.host_wait_ms.clear()
        h2 = eng.submit_block_load("second", source2, dst2)
        waited = eng.host_wait_ms.get("inflight_slot", 0.0)
        still_busy = not busy.query()
    finally:
        gc.enable()
    try:
        assert still_busy, "the busy stream finished before the second submit: the test proves nothing"
        assert waited < 100.0, eng.host_wait_ms
        eng.wait(h2)
        busy.synchronize()
        eng.wait(h1)
        np.testing.assert_array_equal(dst.cpu().numpy().view(np.uint16), want)
        np.testing.assert_array_equal(dst2.cpu().numpy().view(np.uint16), want2)
    finally:
        busy.synchronize()
        eng.shutdown()
        pool.shutdown()
