"""Runtime configuration (same fields and defaults as src/stagehand/config.py:9-46).

``copy_stream_priority`` is accepted for compatibility but every stream this
package creates runs at the default priority (mixed-priority streams have hung
on the target platform).
"""
from __future__ import annotations

from dataclasses import dataclass

__all__ = ["StagehandConfig"]


@dataclass
class StagehandConfig:
    stagehand_enabled: bool = True
    # host pinned pool
    pinned_pool_mb: int = 8192
    pinned_slab_mb: int = 256
    pinned_slab_alignment: int = 512
    # VRAM watermarks (torch.cuda.memory_allocated, MB)
    vram_high_watermark_mb: int = 22000
    vram_low_watermark_mb: int = 18000
    # transfers
    max_inflight_transfers: int = 2
    copy_stream_priority: int = -1
    # keep each file/SquareQ block's source bytes in a pinned host image after
    # its first load, so later loads are a single DMA (no staging copy); costs
    # host memory equal to the streamed bytes of all such blocks
    pinned_source_cache: bool = False
    # how safetensors-backed parameters are read on the device path (and by the
    # VMM backend's region fills):
    # "mmap"   — through a mapping of the file, one host view per tensor, as the
    #            reference does (src/stagehand/scheduler.py:184-241, 564-601);
    #            every 4 KiB page of a fresh mapping faults on first touch;
    # "pread"  — the native reader: each tensor's byte range is read into the
    #            pinned slab on the copy threads, from the page cache where it
    #            holds the file, else in sequential runs from storage; the file
    #            stays in the page cache for later steps, and no mapping is held
    #            (measured on a 12B DiT: as fast as "mmap", warm or cold);
    # "direct" — the same around the page cache (O_DIRECT), for weights larger
    #            than host memory or read once: every step reads storage, unless
    #            pinned_source_cache keeps each block's bytes after the first
    #            (then the fastest cold start, and PCIe-bound after it).
    file_reader: str = "pread"
    # module-backed blocks: a frozen parameter (requires_grad False) whose host
    # tensor already has the runtime dtype keeps that tensor while the block is
    # resident, and eviction points the parameter back at it instead of copying
    # the device copy back (the reference copies back every parameter,
    # src/stagehand/scheduler.py:1216-1231, 1348-1366). Off by default: with it
    # on, in-place writes to a frozen parameter on the device are dropped at
    # eviction.
    frozen_host_copies: bool = False
    # where save-back copies (device -> pinned host at eviction) run:
    # "sdma"   — on a system DMA engine (through the HSA runtime): the compute
    #            units keep computing while a block is copied back;
    # "stream" — hipMemcpyAsync on the copy stream, which runs these copies as
    #            kernels on the compute units; the compute kernels beside them
    #            then run many times slower (measured on a 17.8B-parameter
    #            LoRA training step: 1.75 s per step against 1.13 s with "sdma").
    save_back_engine: str = "sdma"
    # a module-backed block whose last load came from its pinned home buffer (the
    # buffer its last whole-block save-back wrote) gets a digest per chunk of
    # save_back_chunk_bytes on the device after the load; its next save-back
    # compares the digests and copies back only the chunks that changed (frozen
    # weights are not copied again). The home buffer ends up holding the device's
    # bytes, as after the reference's full copy-back (scheduler.py:1216-1226); a
    # changed chunk goes unnoticed only if both 64-bit sums of its digest collide
    # (about 2^-128; one changed word is always seen). Needs the "sdma" engine.
    # The digest is a non-cryptographic checksum, not a proof that a chunk is
    # unchanged: a single changed 8-byte word is always seen, but for several
    # changed words the 2^-128 figure is an argument for random changes, not a
    # bound for structured ones. False copies every byte back, as the reference does.
    save_back_changed_chunks: bool = True
    save_back_chunk_bytes: int = 1 << 18
    # what a module-backed block's save-back waits for inside a step:
    # "last_use"    — the block's last hook or gradient accumulation and the
    #                 step's start (the whole queue when a parameter's version
    #                 counter moved since the step began, or the block was loaded
    #                 again after its last hook). Writes that leave the version
    #                 counter alone (through ``param.data``, e.g. from a hook, EMA
    #                 or weight-norm code) queued after the block's last use are
    #                 not waited for, and the host copy can miss them;
    # "whole_queue" — everything queued on the current stream at the eviction,
    #                 as the reference's synchronous ``param.data.to("cpu")``
    #                 (src/stagehand/scheduler.py:1216-1226) sees it. The copy
    #                 engine then waits for the device to reach the host, which
    #                 runs up to max_run_ahead_blocks ahead (config 5: 1208
    #                 against 1071 ms/step, every byte copied back).
    save_back_fence: str = "last_use"
    # device memory that evicted blocks' save-backs in flight may still hold
    # before the eviction loop waits for the oldest of them (None: the gap
    # between the watermarks, so that allocated memory stays under the high
    # watermark plus that gap)
    save_back_backlog_mb: int | None = None
    # the host waits in before_block until the compute of the block this many
    # blocks back has finished on the device (0: never). Loads and waits are
    # device-side, so without a bound the host can queue work for many blocks
    # ahead of the device, and every evicted block still read by queued work
    # keeps its memory; the reference blocks the host in every load instead.
    # 12 was measured best on config 5 (training): with fewer, the host stalls at
    # the forward/backward turn, where the next loads are several resident blocks
    # away, and the copy engine idles (with frozen host copies: 1028 -> 984 ms/step,
    # peak VRAM unchanged); with more, evicted blocks whose save-backs still wait
    # for queued work hold more memory.
    max_run_ahead_blocks: int = 12
    # the same bound in inference. Inference saves nothing back, so the budget
    # already sees every buffer that queued work still holds, and the bound only
    # keeps the host from reaching the next non-resident block early enough to
    # issue its load while the device computes a run of resident blocks. Measured
    # on config 3 (run-ahead 12 / 16 / 24 / 32 / 57: 188 / 181 / 168 / 163 / 159
    # ms/step) and config 4 (211.4 ms/step at 12, 24 and 57), peak VRAM and
    # evictions unchanged; at 57 the host never waited on it.
    max_run_ahead_blocks_inference: int = 64
    # scheduling policy
    policy: str = "static"
    prefetch_window_blocks: int = 3
    eviction_cooldown_steps: int = 2
    # numeric guards
    strict_bf16: bool = True
    fail_on_dtype_promotion: bool = True
    nan_inf_check: bool = True
    # telemetry
    telemetry_enabled: bool = True
    telemetry_interval_steps: int = 10
    telemetry_file: str = "stagehand_telemetry.jsonl"
    # debug
    debug_trace: bool = False
