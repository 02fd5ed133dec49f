"""Benchmark of the weight-streaming data path on one MI355X.

Default workload: the SquareQ dequant microbench —
a packed slab of 128 int8 tensors (3072x3072, 3072x12288, 12288x3072, 3072x1,
1000x77 cycling; 2,210,302,856 elements, 581,032 rows) with per-output-row
fp32 scales, dequantised on the device to bf16 (round to nearest even). A
"step" is one launch over the whole slab with inputs resident in HBM.

Printed JSON line (one, from rank 0):
  value      algorithmic GB/s of the dequant pass (N*(1+2) + R*4 bytes / time)
  roofline   the dequant kernel against the 8 TB/s HBM3E peak, kernel time
             measured with HIP events on the launch stream
  cpu_baseline  the reference's host dequant (the same torch CPU ops as
             src/stagehand/scheduler.py:290-300, restated in oracle/torch_ref.py)
             timed on a bounded sample of the same slab on this host's cores;
             its output is also compared bit for bit with the device output
  cast       the fp32→bf16 unpack variant of the same shapes
  pcie       pinned hipMemcpyAsync H2D bandwidth (1 GiB x 10)

The process runs with GPU_MAX_HW_QUEUES=8 (--hw-queues; HIP reads it when it
starts, so it is set before torch is imported): HIP maps every stream of a
process onto that many hardware queues (4 by default), and the streamed legs
use the compute stream, the block loader's copy and unpack streams and the
transfer engine's copy stream on top of whatever streams earlier legs made.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBPS = 8000.0
METRIC = "dequant GB/s (% HBM peak); streamed weight GB/s + ms/step, 12B INT8 DiT"
TRAFFIC_FILE = REPO / "profiles" / "traffic.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def settle_launches(fn, settle_ms: float, stream) -> dict:
    """Runs fn() back to back for about settle_ms of wall time before a timed leg.

    From an idle GPU the config-2 kernels take 30-50 launches to reach their steady rate: the
    dequant's per-launch time falls from about 1.14 ms to 1.04 ms over its first 20 launches. The
    timed launches therefore follow a settle phase of the same kernel. The first 20 settle
    launches are timed too and reported as the cold-start average, so both figures are visible."""
    if settle_ms <= 0:
        return {"settle_ms": 0}
    _wall, per = time_launches(fn, 20, 0, stream)
    import torch

    t0 = time.perf_counter()
    n = 20
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
    return {"settle_ms": settle_ms, "settle_launches": n, "cold_first20_ms_avg": round(sum(per) / len(per), 5)}


def time_launches(fn, steps: int, warmup: int, stream) -> tuple[float, list[float]]:
    """Runs fn() warmup+steps times; returns (wall ms for the timed steps, per-launch ms)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return wall_ms, [s.elapsed_time(e) for s, e in zip(starts, ends)]


def measured_traffic(kernel: str) -> float | None:
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if one exists."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return float(data[kernel]["hbm_bytes_per_launch"])
    except Exception:
        return None


def pinned_h2d_gbps(reps: int = 10, nbytes: int = 1 << 30, d2h: bool = False) -> float:
    """Pinned hipMemcpyAsync rate (1 GiB x 10), host to device or, with ``d2h``, back."""
    import torch

    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    host.fill_(1)
    dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.Stream()
    src, dst = (dev, host) if d2h else (host, dev)
    with torch.cuda.stream(stream):
        dst.copy_(src, non_blocking=True)
    stream.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(reps):
            dst.copy_(src, non_blocking=True)
    t1.record(stream)
    stream.synchronize()
    return reps * nbytes / (t0.elapsed_time(t1) * 1e-3) / 1e9


def duplex_gbps(nbytes: int = 1 << 30, reps: int = 10) -> dict:
    """Pinned H2D and D2H at the same time on two streams: each direction's rate."""
    import torch

    hs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    ds = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2)]
    torch.cuda.synchronize()
    for i, (st, (a, b)) in enumerate(zip(streams, ev)):
        a.record(st)
        with torch.cuda.stream(st):
            for _ in range(reps):
                if i == 0:
                    ds[0].copy_(hs[0], non_blocking=True)
                else:
                    hs[1].copy_(ds[1], non_blocking=True)
        b.record(st)
    torch.cuda.synchronize()
    return {"h2d_gbps": round(reps * nbytes / (ev[0][0].elapsed_time(ev[0][1]) * 1e-3) / 1e9, 2),
            "d2h_gbps": round(reps * nbytes / (ev[1][0].elapsed_time(ev[1][1]) * 1e-3) / 1e9, 2)}


def d2d_copy_gbps(nbytes: int = 4 << 30, reps: int = 10) -> float:
    import torch

    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    return reps * 2 * nbytes / (s.elapsed_time(e) * 1e-3) / 1e9


def copy_kernel_gbps(nbytes: int = 4 << 30, reps: int = 10) -> float:
    """Read+write ceiling of a 128-bit stream kernel on this device: a byte copy
    through the unpack kernel, timed on the stream it is launched on."""
    import torch

    from stagehand_amd.unpack import KIND_COPY_BYTES, UnpackPlan, make_descs

    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    half = nbytes // 2  # a region's length is a 32-bit field
    plan = UnpackPlan(make_descs([(KIND_COPY_BYTES, 0, 0, 1, half, 0, 0), (KIND_COPY_BYTES, half, half, 1, half, 0, 0)]))
    stream = torch.cuda.current_stream()
    plan.run(a, b, stream=stream)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(reps):
        plan.run(a, b, stream=stream)
    e.record(stream)
    torch.cuda.synchronize()
    plan.close()
    return reps * 2 * nbytes / (s.elapsed_time(e) * 1e-3) / 1e9


def digest_kernel_gbps(nbytes: int = 740 << 20, chunk: int = 1 << 18, reps: int = 20) -> dict:
    """Read rate of the chunk-digest kernel (sh_block_digest; the save-back comparison reads the
    same bytes) on a buffer the size of a config-5 block, timed on its stream."""
    import torch

    from stagehand_amd import _native

    a = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    dig = torch.empty(2 * -(-nbytes // chunk), dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    lib = _native.lib()

    def run():
        _native.check(lib.sh_block_digest(a.data_ptr(), nbytes, chunk, dig.data_ptr(), stream.cuda_stream),
                      "sh_block_digest")

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(reps):
        run()
    e.record(stream)
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    return {"bytes": nbytes, "chunk": chunk, "ms": round(ms, 4), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def host_cores() -> dict:
    """The host cores this process can use: the CPUs it may run on (its affinity set), bounded by
    the cgroup's CPU quota when one is set; ``os.cpu_count()`` (every CPU of the machine) is
    reported beside them. A CPU baseline runs one torch thread per usable core."""
    cpu_count = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = cpu_count
    quota = None
    try:
        text = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if text and text[0] != "max":
            quota = max(1, int(int(text[0]) / int(text[1])))
    except (OSError, ValueError, IndexError):
        pass
    usable = min(affinity, quota) if quota else affinity
    return {"usable": usable, "affinity": affinity, "cgroup_quota": quota, "os_cpu_count": cpu_count}


def _time_median(fn, budget_s: float, reps: int = 5) -> tuple[float, int]:
    fn()  # warm
    times = []
    t_start = time.perf_counter()
    while len(times) < reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def cpu_baseline(regions, src, scales, dst, budget_s: float) -> dict:
    """The reference's host dequant (torch CPU ops) on a bounded sample; bit-checked against dst."""
    import torch

    from oracle.torch_ref import host_dequant_into

    cores = host_cores()
    threads = cores["usable"]
    torch.set_num_threads(threads)
    sample = regions[:10]  # 2 x each shape; ~1/11 of the pass's bytes
    elems = sum(g.numel for g in sample)
    rows = sum(g.rows for g in sample)
    algo = elems * 3 + rows * 4
    host_q = [src[g.elem_off:g.elem_off + g.numel].view(g.rows, g.cols).cpu() for g in sample]
    host_s = [scales[g.scale_off:g.scale_off + g.rows].cpu() for g in sample]
    zeros = [torch.zeros(g.rows, dtype=torch.float32) for g in sample]
    slab = torch.empty(elems * 2, dtype=torch.uint8, pin_memory=True)
    offs, pos = [], 0
    for g in sample:
        offs.append(pos)
        pos += g.numel * 2
    work = [(o, q, s, z, g.rows, g.cols) for o, q, s, z, g in zip(offs, host_q, host_s, zeros, sample)]
    med, runs = _time_median(lambda: host_dequant_into(slab, work), budget_s)
    # parity gate: the device output equals the reference's host computation bit for bit
    dev_bytes = torch.cat([dst[g.elem_off:g.elem_off + g.numel].view(torch.uint8).cpu() for g in sample])
    bit_exact = bool(torch.equal(dev_bytes, slab))
    return {
        "value": round(algo / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"tensors 0-9 of the config-2 slab ({elems} int8 elements, {rows} rows, "
                   f"{algo} algorithmic bytes), torch CPU ops of scheduler.py:290-300 into a pinned slab, "
                   f"median of {runs} runs, {threads} torch threads"),
        "ms_per_sample": round(med * 1e3, 2),
        "bit_exact_vs_device": bit_exact,
        "host_cores": cores,
    }


def cpu_cast_baseline(regions, csrc, dst, budget_s: float) -> dict:
    """The reference's host fp32→bf16 pack (``region.copy_(param.to(bf16))``, scheduler.py:1066-1071
    and 168-181) on a bounded sample of the config-2 cast variant; bit-checked against dst."""
    import torch

    from oracle.torch_ref import host_cast_into

    cores = host_cores()
    threads = cores["usable"]
    torch.set_num_threads(threads)
    sample = regions[:10]
    elems = sum(g.numel for g in sample)
    algo = elems * 6
    params = [csrc[g.elem_off:g.elem_off + g.numel].view(g.rows, g.cols).cpu() for g in sample]
    slab = torch.empty(elems * 2, dtype=torch.uint8, pin_memory=True)
    work, pos = [], 0
    for g, p in zip(sample, params):
        work.append((pos, p))
        pos += g.numel * 2
    med, runs = _time_median(lambda: host_cast_into(slab, work), budget_s)
    dev_bytes = torch.cat([dst[g.elem_off:g.elem_off + g.numel].view(torch.uint8).cpu() for g in sample])
    return {
        "value": round(algo / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"tensors 0-9 of the config-2 fp32 slab ({elems} elements, {algo} algorithmic bytes), "
                   f"torch CPU ops of scheduler.py:1066-1071 into a pinned slab, median of {runs} runs, "
                   f"{threads} torch threads"),
        "ms_per_sample": round(med * 1e3, 2),
        "bit_exact_vs_device": bool(torch.equal(dev_bytes, slab)),
    }


def cpu_reference_config4_step(seed: int) -> dict:
    """The reference's config-4 block load timed on a sample: for one double-stream and one
    single-stream block of the 12B DiT, the torch CPU dequant of every Linear into a pinned bf16
    slab (scheduler.py:290-300) and the bias copies, then the bf16 H2D and its wait, one block after
    another as the reference's hook thread does (scheduler.py:953-1031, 1089-1120). The step is
    scaled from the two blocks (19 double + 38 single); synthetic int8 values of the DiT's shapes."""
    import torch

    from oracle.torch_ref import host_dequant_into
    from bench_workloads import FluxStyleDiT, dit_linear_layers

    threads = host_cores()["usable"]
    torch.set_num_threads(threads)
    with torch.device("meta"):
        model = FluxStyleDiT(depth_double=1, depth_single=1)
    g = torch.Generator().manual_seed(seed)
    out: dict = {"cores": threads, "kind": "port"}
    for kind in ("double_blocks.0", "single_blocks.0"):
        lins = [(n, m) for n, m in dit_linear_layers(model) if n.startswith(kind + ".")]
        work, biases, pos = [], [], 0
        for _n, lin in lins:
            o, i = lin.out_features, lin.in_features
            q = torch.randint(-127, 128, (o, i), dtype=torch.int8, generator=g)
            sc = torch.exp(torch.randn(o, generator=g) * 0.5 - 6.0)
            work.append((pos, q, sc, torch.zeros(o), o, i))
            pos += o * i * 2
            biases.append((pos, (torch.randn(o, generator=g) * 0.02).to(torch.bfloat16)))
            pos += o * 2
        slab = torch.empty(pos, dtype=torch.uint8, pin_memory=True)
        dev = torch.empty(pos, dtype=torch.uint8, device="cuda")
        times = []
        for _rep in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            host_dequant_into(slab, work)
            for off, b in biases:
                slab[off:off + b.numel() * 2].copy_(b.view(torch.uint8))
            t1 = time.perf_counter()
            dev.copy_(slab, non_blocking=True)
            torch.cuda.synchronize()
            times.append((t1 - t0, time.perf_counter() - t1))
        host_s, h2d_s = sorted(times)[1]
        out[kind.split(".")[0]] = {"bf16_bytes": pos, "host_dequant_ms": round(host_s * 1e3, 1),
                                   "h2d_ms": round(h2d_s * 1e3, 1)}
        del slab, dev, work
    d, sg = out["double_blocks"], out["single_blocks"]
    step = 19 * (d["host_dequant_ms"] + d["h2d_ms"]) + 38 * (sg["host_dequant_ms"] + sg["h2d_ms"])
    out["ms_per_step"] = round(step, 1)
    out["pcie_bytes_per_step"] = 19 * d["bf16_bytes"] + 38 * sg["bf16_bytes"]
    out["sample"] = ("one double- and one single-stream block of the 12B DiT (synthetic int8, fp32 row scales), "
                     "median of 3; step = 19 double + 38 single")
    return out


def cpu_reference_config3_step(src: Path) -> dict:
    """The reference's config-3 block load timed on a sample: for one double-stream and one
    single-stream shard, ``copy_`` of every tensor from a ``torch.frombuffer`` view of the mapped
    file into a pinned slab (scheduler.py:184-241, 564-601; the mapping stays open and warm across
    loads, as the reference caches it), then the bf16 H2D and its wait (transfer.py:108-143,
    scheduler.py:1089-1120). Scaled to 19 + 38 blocks."""
    import mmap
    import warnings

    import torch

    from stagehand_amd.registry import parse_safetensors_index

    threads = host_cores()["usable"]
    torch.set_num_threads(threads)
    out: dict = {"cores": threads, "kind": "reference ops (torch)"}
    for kind in ("double_blocks", "single_blocks"):
        path = src / f"{kind}.0.safetensors"
        index = parse_safetensors_index(path)
        with open(path, "rb") as fh:
            mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
            view = memoryview(mm)
            with warnings.catch_warnings():
                warnings.simplefilter("ignore", UserWarning)
                tensors = [torch.frombuffer(view[o:o + n], dtype=dt) for o, n, dt, _shape in index.values()]
            total = sum(t.numel() * t.element_size() for t in tensors)
            slab = torch.empty(total, dtype=torch.uint8, pin_memory=True)
            dev = torch.empty(total, dtype=torch.uint8, device="cuda")
            times = []
            for _rep in range(4):  # the first pass maps the pages; the rest are the steady state
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                pos = 0
                for t in tensors:
                    n = t.numel() * t.element_size()
                    slab[pos:pos + n].view(t.dtype).copy_(t)
                    pos += n
                t1 = time.perf_counter()
                dev.copy_(slab, non_blocking=True)
                torch.cuda.synchronize()
                times.append((t1 - t0, time.perf_counter() - t1))
            first = times[0]
            stage_s, h2d_s = sorted(times[1:])[1]
            out[kind] = {"bf16_bytes": total, "stage_ms": round(stage_s * 1e3, 1), "h2d_ms": round(h2d_s * 1e3, 1),
                         "first_stage_ms": round(first[0] * 1e3, 1)}
            del tensors, slab, dev, t  # every view of the mapping, before it is closed
            view.release()
            mm.close()
    d, sg = out["double_blocks"], out["single_blocks"]
    serial = 19 * (d["stage_ms"] + d["h2d_ms"]) + 38 * (sg["stage_ms"] + sg["h2d_ms"])
    overlap = max(19 * d["stage_ms"] + 38 * sg["stage_ms"], 19 * d["h2d_ms"] + 38 * sg["h2d_ms"])
    out["ms_per_step_serial"] = round(serial, 1)
    out["ms_per_step_overlapped"] = round(overlap, 1)
    out["pcie_bytes_per_step"] = 19 * d["bf16_bytes"] + 38 * sg["bf16_bytes"]
    out["sample"] = ("shards double_blocks.0 and single_blocks.0 of the config-3 files, page cache warm, mapping "
                     "warm; median of 3 after a first pass; step = 19 double + 38 single, serial (the reference "
                     "stages on the hook thread) and with staging fully overlapped with the H2D")
    return out


def _dit_inputs(seed: int, img_tokens: int = 4096, txt_tokens: int = 512, hidden: int = 3072):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    img = torch.randn(1, img_tokens, hidden, device="cuda", generator=g).to(torch.bfloat16)
    txt = torch.randn(1, txt_tokens, hidden, device="cuda", generator=g).to(torch.bfloat16)
    vec = torch.randn(1, hidden, device="cuda", generator=g).to(torch.bfloat16)
    return img, txt, vec


def _dit_config(kind: str, args, pinned: bool, reader: str = "mmap"):
    import stagehand_amd as stagehand

    if kind.startswith("squareq"):
        # 6 GB steady-state cap: the high watermark leaves room for the prefetch
        # window's blocks and their int8 staging buffers on top of it (measured:
        # window 2, watermarks 3.8 / 2.8 GB keep the peak under 6 GB while the
        # loads still run ahead of compute)
        high, low = (int(v) for v in getattr(args, "squareq_watermarks", "3800,2800").split(","))
        cfg = stagehand.StagehandConfig(pinned_pool_mb=2048, pinned_slab_mb=256, vram_high_watermark_mb=high,
                                        vram_low_watermark_mb=low, prefetch_window_blocks=args.dit_prefetch,
                                        max_inflight_transfers=args.dit_prefetch + 1, nan_inf_check=False,
                                        strict_bf16=False, telemetry_enabled=True, pinned_source_cache=pinned)
    else:
        # 24 GB VRAM budget with the layer-mode convention (high 80 %, low 60 %,
        # src/stagehand/layer.py:145-147): part of the 23.7 GB model stays resident,
        # the rest streams every step
        cfg = stagehand.StagehandConfig(pinned_pool_mb=4096, pinned_slab_mb=256, vram_high_watermark_mb=19200,
                                        vram_low_watermark_mb=14400, prefetch_window_blocks=2,
                                        max_inflight_transfers=3, nan_inf_check=False, strict_bf16=False,
                                        telemetry_enabled=True, pinned_source_cache=pinned, file_reader=reader)
    if getattr(args, "run_ahead", None) is not None:
        cfg.max_run_ahead_blocks = args.run_ahead
        cfg.max_run_ahead_blocks_inference = args.run_ahead
    cfg.telemetry_file = None
    return cfg


def _dit_model():
    import torch

    from bench_workloads import FluxStyleDiT, materialize_norms_

    with torch.device("meta"):
        model = FluxStyleDiT()
    model.requires_grad_(False)  # frozen base weights: eligible for file / SquareQ backing
    materialize_norms_(model)
    return model


def _union(intervals: list[tuple[float, float]]) -> list[tuple[float, float]]:
    out: list[list[float]] = []
    for a, b in sorted(intervals):
        if out and a <= out[-1][1]:
            out[-1][1] = max(out[-1][1], b)
        else:
            out.append([a, b])
    return [(a, b) for a, b in out]


def _length(iv: list[tuple[float, float]]) -> float:
    return sum(b - a for a, b in iv)


def _intersect(x: list[tuple[float, float]], y: list[tuple[float, float]]) -> float:
    i = j = 0
    tot = 0.0
    while i < len(x) and j < len(y):
        a, b = max(x[i][0], y[j][0]), min(x[i][1], y[j][1])
        if b > a:
            tot += b - a
        if x[i][1] < y[j][1]:
            i += 1
        else:
            j += 1
    return tot


def load_gap_causes(trace: dict, top: int = 6) -> list[dict]:
    """For the longest gaps between consecutive block loads of a traced step (one copy's end to the
    next copy's start): when the next load was submitted by the host relative to the gap, and the
    host waits (``AsyncTransferEngine.host_wait``) that overlapped the gap before that submit."""
    loads = sorted(trace["loads"], key=lambda l: l[2])
    waits = trace.get("host_waits") or []
    gaps = []
    for a, b in zip(loads, loads[1:]):
        g0, g1 = a[3], b[2]
        if g1 - g0 <= 1.0:
            continue
        submit = b[5] if len(b) > 5 else None
        until = min(g1, submit) if submit is not None else g1
        by_kind: dict[str, float] = {}
        for kind, w0, w1 in waits:
            ov = min(w1, until) - max(w0, g0)
            if ov > 0:
                by_kind[kind] = round(by_kind.get(kind, 0.0) + ov, 2)
        gaps.append({"gap_ms": round(g1 - g0, 2), "at_ms": round(g0, 1), "next_block": b[0],
                     "submitted_ms_after_gap_start": None if submit is None else round(submit - g0, 2),
                     "host_waits_before_submit_ms": by_kind})
    return sorted(gaps, key=lambda g: -g["gap_ms"])[:top]


def timeline_stats(trace: dict, pcie_peak_gbps: float | None) -> dict:
    """Copy / compute busy time and their overlap over one traced step (device timestamps)."""
    loads, comp = trace["loads"], trace["compute"]
    if not loads or not comp:
        return {}
    span0 = min(min(l[2] for l in loads), min(c[1] for c in comp))
    span1 = max(max(l[4] for l in loads), max(c[2] for c in comp))
    copy_iv = _union([(l[2], l[3]) for l in loads])
    comp_iv = _union([(c[1], c[2]) for c in comp])
    copy_ms, comp_ms = _length(copy_iv), _length(comp_iv)
    nbytes = sum(l[1] for l in loads)
    res = {
        "step_span_ms": round(span1 - span0, 2),
        "copy_busy_ms": round(copy_ms, 2),
        "compute_busy_ms": round(comp_ms, 2),
        "copy_compute_overlap_ms": round(_intersect(copy_iv, comp_iv), 2),
        "compute_hidden_frac": round(_intersect(copy_iv, comp_iv) / comp_ms, 4) if comp_ms else None,
        "copy_busy_frac": round(copy_ms / (span1 - span0), 4),
        "h2d_gbps_while_copying": round(nbytes / (copy_ms * 1e-3) / 1e9, 2),
        "loads": len(loads),
    }
    if pcie_peak_gbps:
        res["h2d_frac_of_measured_pcie_while_copying"] = round(res["h2d_gbps_while_copying"] / pcie_peak_gbps, 4)
    d2h = trace.get("d2h") or []
    if d2h:
        d2h_iv = _union([(a, b) for _n, a, b, *_k in d2h])
        d2h_ms = _length(d2h_iv)
        res["d2h_busy_ms"] = round(d2h_ms, 2)
        res["d2h_busy_frac"] = round(d2h_ms / (span1 - span0), 4)
        res["d2h_gbps_while_copying"] = round(sum(d[0] for d in d2h) / (d2h_ms * 1e-3) / 1e9, 2) if d2h_ms else None
        res["d2h_h2d_overlap_ms"] = round(_intersect(d2h_iv, copy_iv), 2)
        res["d2h_span_ms"] = [round(min(d[1] for d in d2h) - span0, 1), round(max(d[2] for d in d2h) - span0, 1)]
    waits = trace.get("host_waits") or []
    if waits:
        res["host_waits"] = len(waits)
        res["host_wait_ms"] = round(sum(b - a for _k, a, b in waits), 2)
    return res


def _file_weight_check(rt) -> dict:
    """Every file-backed parameter of every resident block of a config-3 runtime: its bytes in the
    block buffer against its bytes in the shard. The reference stages a bf16 tensor of a
    safetensors file as a byte copy into the block's layout (scheduler.py:184-241), so the
    buffer must hold the file's bytes exactly. Module-resident parameters (norm weights) are
    views of the buffer and are counted apart."""
    import numpy as np
    import torch

    maps: dict[str, np.memmap] = {}
    blocks = params = module_params = 0
    nbytes = 0
    exact = True
    for e in rt.registry.blocks_in_order():
        buf = rt.residency.get_entry(e.block_id).gpu_tensor
        if buf is None:
            continue
        host = buf.detach().view(torch.uint8).cpu().numpy()
        specs = {f.param_name: f for f in e.file_param_specs}
        for name, _shape, _dtype, off, numel in e.param_layout:
            f = specs.get(name)
            if f is None:
                module_params += 1
                continue
            if f.file_path not in maps:
                maps[f.file_path] = np.memmap(f.file_path, dtype=np.uint8, mode="r")
            n = int(f.source_nbytes)
            exact &= n == 2 * int(numel) and bool(np.array_equal(host[off:off + n], maps[f.file_path][f.file_offset:f.file_offset + n]))
            params += 1
            nbytes += n
        blocks += 1
    return {"resident_blocks_checked": blocks, "file_params_checked": params, "module_params": module_params,
            "bytes_checked": nbytes, "bit_exact": bool(exact)}


def _dit_run(kind: str, args, src: Path, layers, pinned: bool, reader: str = "mmap") -> dict:
    import torch

    import stagehand_amd as stagehand
    from bench_workloads import DIT_BLOCK_PATTERN, dit_forward_flops, dit_linear_layers

    model = _dit_model()  # a fresh module tree per runtime: conversion drops the module's weights

    rt = stagehand.StagehandRuntime(model, _dit_config(kind, args, pinned, reader), block_pattern=DIT_BLOCK_PATTERN,
                                    dtype=torch.bfloat16, inference_mode=True)
    if kind == "squareq_v2":
        converted = rt.convert_registry_to_squareq_v2_backed(str(src), str(src.with_suffix(".manifest.json")))
    elif kind == "squareq":
        converted = rt.convert_registry_to_file_backed(str(src))
    else:
        converted = rt.convert_registry_to_file_backed_sharded(str(src))
    img, txt, vec = _dit_inputs(args.seed)
    bf16_bytes = sum(e.size_bytes for e in rt.registry.blocks_in_order())

    def step(i: int):
        rt.begin_step(i)
        with torch.no_grad(), rt.managed_forward():
            out = model(img, txt, vec)
        rt.end_step()
        return out

    for i in range(args.dit_warmup):
        step(i)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    b0 = rt.engine.bytes_h2d
    rt.engine.host_wait_ms.clear()
    trace_marker(args)
    t1 = time.perf_counter()
    for i in range(args.dit_steps):
        out = step(args.dit_warmup + i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t1
    trace_marker(args)
    sent = rt.engine.bytes_h2d - b0
    ms = wall / args.dit_steps * 1e3
    hist = rt.telemetry.history[-args.dit_steps:]
    host_waits = {k: round(v / args.dit_steps, 1) for k, v in sorted(rt.engine.host_wait_ms.items())}
    # one more step with device timing of every load and compute span (not part of the timed steps)
    rt.engine.start_trace()
    step(args.dit_warmup + args.dit_steps)
    trace = rt.engine.stop_trace()
    timeline = timeline_stats(trace, getattr(args, "pcie_peak_gbps", None))
    if trace["loads"]:
        timeline["load_gap_causes"] = load_gap_causes(trace)
    check = None
    if layers is not None:
        # every Linear of every resident block: its streamed weight and bias against the torch
        # device expression of the reference's host dequant (scheduler.py:290-308) on its payload
        n_layers, exact = 0, True
        for e in rt.registry.blocks_in_order():
            if rt.residency.get_entry(e.block_id).gpu_tensor is None:
                continue
            for n, lin in e.module_ref().named_modules():
                if not isinstance(lin, torch.nn.Linear):
                    continue
                L = layers[f"{e.block_id}.{n}"]
                want = ((L["qweight"].cuda().to(torch.float32) - L["zero_point"].cuda().unsqueeze(1))
                        * L["scale"].cuda().unsqueeze(1)).to(torch.bfloat16)
                exact &= bool(torch.equal(lin.weight.view(torch.int16), want.view(torch.int16)))
                exact &= bool(torch.equal(lin.bias.view(torch.int16), L["bias"].cuda().to(torch.bfloat16).view(torch.int16)))
                n_layers += 1
        check = {"resident_layers_checked": n_layers, "bit_exact": exact}
    elif kind == "file":
        check = _file_weight_check(rt)
    res = {
        "source_mode": "pinned source images" if pinned else "bounded pinned pool (staged)",
        "file_reader": reader if kind in ("file", "squareq_v2") else None,
        "params_converted": converted,
        "int8_elements": (sum(l.in_features * l.out_features for _n, l in dit_linear_layers(model))
                          if kind.startswith("squareq") else None),
        "scale_rows": sum(l.out_features for _n, l in dit_linear_layers(model)) if kind.startswith("squareq") else None,
        "block_bf16_bytes_per_step": bf16_bytes,
        "pcie_bytes_per_step": sent // args.dit_steps,
        "ms_per_step": round(ms, 2),
        "streamed_gbps": round(sent / args.dit_steps / (ms * 1e-3) / 1e9, 2),
        "bf16_weight_gbps": round(bf16_bytes / (ms * 1e-3) / 1e9, 2),
        "forward_tflop": round(dit_forward_flops(model, 4096, 512) / 1e12, 2),
        "steps": args.dit_steps,
        "warmup": args.dit_warmup,
        "peak_vram_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2),
        "pinned_image_gb": round(rt.engine.pinned_image_bytes / 1e9, 2),
        "stall_ms_per_step": round(sum(m.stall_time_ms for m in hist) / len(hist), 2),
        "evictions_per_step": sum(m.evictions for m in hist) / len(hist),
        "host_wait_ms_per_step": host_waits,
        "weight_check": check,
        "out_finite": bool(torch.isfinite(out.float()).all()),
        "timeline": timeline,
    }
    rt.shutdown()
    # drop every device buffer of this runtime before the next measurement (the
    # budget counts all of torch's allocations)
    for e in rt.registry.blocks_in_order():
        rt.residency.get_entry(e.block_id).gpu_tensor = None
    del rt, model, out, img, txt, vec
    import gc

    gc.collect()
    torch.cuda.empty_cache()
    return res


def trace_marker(args) -> None:
    """With ``--trace-markers``: one allocation-free unpack of 16 zero bytes, whose
    ``sh_put_descs_kernel`` launch runs nowhere else in a streamed step. Placed before and after the
    timed steps, the two launches bound them in a rocprofv3 kernel trace (``--trace-summary``)."""
    if not getattr(args, "trace_markers", False):
        return
    import torch

    from stagehand_amd.unpack import KIND_ZERO_BYTES, make_descs, unpack_noalloc

    buf = torch.empty(16, dtype=torch.uint8, device="cuda")
    unpack_noalloc(make_descs([(KIND_ZERO_BYTES, 0, 0, 1, 16, 0, 0)]), None, buf)
    torch.cuda.synchronize()


def trace_summary(trace_dir: Path, h2d_bytes: int | None, pcie_gbps: float | None) -> dict:
    """Copy/compute overlap of the marked steps in rocprofv3 CSVs (``--kernel-trace
    --memory-copy-trace --output-format csv``): the window runs from the end of the first
    ``sh_put_descs_kernel`` dispatch to the start of the last. Within it: the union of
    host-to-device copy intervals, of the unpack kernels (``sh_*``) and of all other kernels
    (the model's compute), their intersection, and, given the window's H2D bytes (the bench's
    ``pcie_bytes_per_step`` times its steps), the H2D rate while copying.

    A kernel trace alone (no ``memory_copy_trace.csv``) gives the compute side and the block
    arrivals: each block load ends with its unpack kernel, launched once the block's bytes have
    landed, so the unpack kernels' start times are the blocks' arrival times. Reported: compute
    busy over the window, its longest idle stretches, and the arrival intervals; with the
    window's H2D bytes, the H2D rate over the window."""
    import csv

    def rows(pattern: str, required: bool = True) -> list[dict]:
        files = sorted(trace_dir.rglob(pattern))
        if not files:
            if not required:
                return []
            raise FileNotFoundError(f"no {pattern} under {trace_dir}")
        with open(files[0], newline="") as fh:
            return list(csv.DictReader(fh))

    kernels = rows("*kernel_trace.csv")
    copies = rows("*memory_copy_trace.csv", required=False)
    copy_trace = bool(copies) or bool(sorted(trace_dir.rglob("*memory_copy_trace.csv")))
    marks = sorted((int(k["Start_Timestamp"]), int(k["End_Timestamp"])) for k in kernels
                   if k["Kernel_Name"].startswith("sh_put_descs_kernel"))
    if len(marks) < 2:
        raise ValueError("the trace has fewer than two marker dispatches (run the bench with --trace-markers)")
    w0, w1 = marks[0][1], marks[-1][0]

    def clip(iv):
        return [(max(a, w0), min(b, w1)) for a, b in iv if b > w0 and a < w1]

    marker_names = ("sh_put_descs_kernel", "sh_fill_tile_map_kernel")
    unpack, compute = [], []
    for k in kernels:
        name = k["Kernel_Name"]
        if name.startswith(marker_names):
            continue
        iv = (int(k["Start_Timestamp"]), int(k["End_Timestamp"]))
        (unpack if name.startswith("sh_") else compute).append(iv)
    h2d = [(int(c["Start_Timestamp"]), int(c["End_Timestamp"])) for c in copies
           if c["Direction"].endswith("HOST_TO_DEVICE")]
    d2h = [(int(c["Start_Timestamp"]), int(c["End_Timestamp"])) for c in copies
           if c["Direction"].endswith("DEVICE_TO_HOST")]
    h2d_w, d2h_w, comp_w, unp_w = (_union(clip(x)) for x in (h2d, d2h, compute, unpack))
    ms = 1e-6
    window_ms = (w1 - w0) * ms
    if not copy_trace:
        import statistics

        starts = sorted(a for a, b in unpack if w0 <= a < w1)
        gaps = [(b - a) * ms for a, b in zip(starts, starts[1:])]
        idle = sorted(((b0 - a1) * ms for (_a0, a1), (b0, _b1) in zip(comp_w, comp_w[1:])), reverse=True)
        comp_busy = _length(comp_w) * ms
        out = {
            "window_ms": round(window_ms, 2),
            "compute_kernels": sum(1 for a, b in compute if b > w0 and a < w1),
            "compute_busy_ms": round(comp_busy, 2),
            "compute_busy_frac": round(comp_busy / window_ms, 4) if window_ms else None,
            "compute_idle_top_ms": [round(x, 2) for x in idle[:5]],
            "unpack_kernels": len(starts),
            "unpack_busy_ms": round(_length(unp_w) * ms, 2),
            "arrival_interval_ms": ({"median": round(statistics.median(gaps), 3), "min": round(min(gaps), 3),
                                     "max": round(max(gaps), 3)} if gaps else None),
        }
        if h2d_bytes:
            out["h2d_bytes"] = int(h2d_bytes)
            out["h2d_gbps_over_window"] = round(h2d_bytes / (window_ms * 1e-3) / 1e9, 2)
            if pcie_gbps:
                out["frac_of_measured_pinned_pcie_over_window"] = round(out["h2d_gbps_over_window"] / pcie_gbps, 4)
        return out
    h2d_busy = _length(h2d_w) * ms
    comp_busy = _length(comp_w) * ms
    overlap = _intersect(h2d_w, comp_w) * ms
    out = {
        "window_ms": round(window_ms, 2),
        "h2d_copies": sum(1 for a, b in h2d if b > w0 and a < w1),
        "h2d_busy_ms": round(h2d_busy, 2),
        "h2d_busy_frac": round(h2d_busy / window_ms, 4) if window_ms else None,
        "d2h_busy_ms": round(_length(d2h_w) * ms, 2),
        "compute_kernels": sum(1 for a, b in compute if b > w0 and a < w1),
        "compute_busy_ms": round(comp_busy, 2),
        "unpack_kernels": sum(1 for a, b in unpack if b > w0 and a < w1),
        "unpack_busy_ms": round(_length(unp_w) * ms, 2),
        "h2d_compute_overlap_ms": round(overlap, 2),
        "compute_hidden_frac": round(overlap / comp_busy, 4) if comp_busy else None,
    }
    if h2d_bytes:
        out["h2d_bytes"] = int(h2d_bytes)
        out["h2d_gbps_while_copying"] = round(h2d_bytes / (h2d_busy * 1e-3) / 1e9, 2) if h2d_busy else None
        out["h2d_gbps_over_window"] = round(h2d_bytes / (window_ms * 1e-3) / 1e9, 2)
        if pcie_gbps and out["h2d_gbps_while_copying"]:
            out["frac_of_measured_pinned_pcie_while_copying"] = round(out["h2d_gbps_while_copying"] / pcie_gbps, 4)
    return out


def kernel_stats(trace_dir: Path, last: int) -> dict:
    """Per-kernel dispatch statistics of a rocprofv3 ``--kernel-trace`` CSV for the library's kernels
    (``sh_*``), over the last ``last`` dispatches of each kernel (the bench's timed launches, after
    its settle and warm-up launches), in µs."""
    import csv
    import statistics

    files = sorted(trace_dir.rglob("*kernel_trace.csv"))
    if not files:
        raise FileNotFoundError(f"no kernel_trace.csv under {trace_dir}")
    per: dict[str, list[tuple[int, float]]] = {}
    with open(files[0], newline="") as fh:
        for row in csv.DictReader(fh):
            name = row["Kernel_Name"]
            if name.startswith("sh_"):
                per.setdefault(name, []).append((int(row["Start_Timestamp"]),
                                                 (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3))
    out = {}
    for name, rows in sorted(per.items()):
        d = [us for _t, us in sorted(rows)][-last:]
        if d:
            out[name] = {"calls": len(d), "avg_us": round(statistics.fmean(d), 2), "min_us": round(min(d), 2),
                         "max_us": round(max(d), 2), "median_us": round(statistics.median(d), 2)}
    return out


def pmc_summary(dirs: list[Path]) -> dict:
    """Per-kernel medians of every counter in rocprofv3 ``--pmc`` CSVs (``*counter_collection.csv``
    under each directory), for the library's kernels (names starting with ``sh_``), with the
    kernels' median dispatch durations in ns."""
    import csv
    import statistics

    vals: dict[str, dict[str, list[float]]] = {}
    for d in dirs:
        for f in sorted(Path(d).rglob("*counter_collection.csv")):
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    name = row["Kernel_Name"]
                    if not name.startswith("sh_"):
                        continue
                    k = vals.setdefault(name, {})
                    k.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
                    k.setdefault("_duration_ns", []).append(float(row["End_Timestamp"]) - float(row["Start_Timestamp"]))
    return {name: {c: statistics.median(v) for c, v in sorted(cs.items())} for name, cs in sorted(vals.items())}


def _dit_host_bf16(seed: int):
    """The 12B DiT with every block parameter in host memory as bf16: N(0, 0.02)
    drawn on the device (fast), RMSNorm weights ones; frozen."""
    import torch

    from bench_workloads import FluxStyleDiT

    with torch.device("meta"):
        model = FluxStyleDiT()
    g = torch.Generator(device="cuda").manual_seed(seed)
    for mod in model.modules():
        for name, prm in list(mod.named_parameters(recurse=False)):
            if isinstance(mod, torch.nn.RMSNorm):
                t = torch.ones(prm.shape, dtype=torch.bfloat16)
            else:
                t = (torch.randn(prm.shape, device="cuda", generator=g) * 0.02).to(torch.bfloat16).cpu()
            setattr(mod, name, torch.nn.Parameter(t, requires_grad=False))
    return model


def turbo_leg(args) -> dict:
    """The config-3 DiT (bf16, 23.7 GB of blocks) through the turbo window engine:
    every block pinned on the host, a window of 3 device slots, one H2D per block
    per step. Run in the engine's own layout (contiguous slots, no write-back of
    frozen blocks) and in the reference's layout (a slot tensor per parameter,
    write-back of every evicted block), its write-backs of changed chunks and of
    every byte."""
    import gc

    import torch

    from stagehand_amd.turbo import TurboConductor
    from bench_workloads import DIT_BLOCK_PATTERN, dit_forward_flops

    img, txt, vec = _dit_inputs(args.seed)
    out = {"workload": "config3 bf16 Flux-style DiT (19 double + 38 single blocks, 11.84 B params), module-backed "
                       "weights pinned on the host, turbo window of 3 slots, 4096 image + 512 text tokens, inference"}
    # the reference layout writes every evicted block back (engine.rs:232-262): by default only the
    # chunks changed on the device cross PCIe (the host regions end up the same); then every byte
    legs = (("engine_layout", True, "auto", 1 << 18), ("reference_layout", False, "always", 1 << 18),
            ("reference_layout_full_write_back", False, "always", 0))
    for label, contiguous, wb, chunk in legs:
        t0 = time.perf_counter()
        model = _dit_host_bf16(args.seed)
        flops = dit_forward_flops(model, 4096, 512)
        cond = TurboConductor(model, block_pattern=DIT_BLOCK_PATTERN, dtype=torch.bfloat16,
                              contiguous_slots=contiguous, writeback=wb, writeback_chunk_bytes=chunk)
        cond.prepare()
        gc.collect()
        prep_s = time.perf_counter() - t0
        handles = cond.install_hooks()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()

        def step():
            with torch.no_grad():
                return model(img, txt, vec)

        for _ in range(args.dit_warmup):
            step()
        torch.cuda.synchronize()
        h0, d0 = cond.engine.bytes_moved()
        t1 = time.perf_counter()
        for _ in range(args.dit_steps):
            y = step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t1
        h1, d1 = cond.engine.bytes_moved()
        cond.start_trace()
        step()
        timeline = timeline_stats(cond.stop_trace(), getattr(args, "pcie_peak_gbps", None))
        ms = wall / args.dit_steps * 1e3
        h2d = (h1 - h0) // args.dit_steps
        res = {"ms_per_step": round(ms, 2), "h2d_bytes_per_step": h2d, "d2h_bytes_per_step": (d1 - d0) // args.dit_steps,
               "h2d_gbps": round(h2d / (ms * 1e-3) / 1e9, 2), "forward_tflop": round(flops / 1e12, 2),
               "peak_vram_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2), "prepare_s": round(prep_s, 1),
               "out_finite": bool(torch.isfinite(y.float()).all()), "steps": args.dit_steps, "warmup": args.dit_warmup,
               "timeline": timeline}
        if getattr(args, "pcie_peak_gbps", None):
            res["pcie_frac"] = round(res["h2d_gbps"] / args.pcie_peak_gbps, 4)
        out[label] = res
        log(f"turbo/{label}: {res}")
        for h in handles:
            h.remove()
        cond.shutdown(restore_params=False)
        del cond, model, y
        gc.collect()
        torch.cuda.empty_cache()
    return out


def train_leg(args) -> dict:
    """Config 5: one training step of a 48-block hidden-4096 DiT (17.8 B bf16 weights,
    frozen, module-backed; LoRA rank 32 on the self-attention projections, trainable)
    streamed through StagehandRuntime block mode under a 24 GB VRAM budget (watermarks
    80 / 60 %), prefetch window 3, forward + backward hooks, activation checkpointing
    per block, MSE loss, SGD on the LoRA weights. Run with the reference's eviction
    (every parameter copied back to the host) and with frozen host copies (only the
    trainable parameters copied back)."""
    import gc

    import torch

    import stagehand_amd as stagehand
    from bench_workloads import TRAIN_BLOCK_PATTERN, TrainDiT, init_train_dit_

    g = torch.Generator(device="cuda").manual_seed(args.seed + 5)
    x = torch.randn(1, 4096, 4096, device="cuda", generator=g).to(torch.bfloat16)
    ctx = torch.randn(1, 512, 4096, device="cuda", generator=g).to(torch.bfloat16)
    vec = torch.randn(1, 4096, device="cuda", generator=g).to(torch.bfloat16)
    target = torch.randn(1, 4096, 4096, device="cuda", generator=g)
    out = {"workload": "config5 48-block DiT (hidden 4096, 32 heads, MLP 4, self + cross attention, 17.77 B frozen "
                       "bf16 block weights, LoRA r32 on self-attention q/k/v/o = 50.3 M trainable), batch 1 x 4096 "
                       "tokens + 512 conditioning tokens, MSE loss, SGD on LoRA, activation checkpointing, "
                       "VRAM budget 24 GB (watermarks 19200 / 14400 MB), prefetch window 3"}
    # (label, frozen_host_copies, save_back_changed_chunks): the reference's eviction copies every
    # parameter back; by default only the chunks changed since the load cross PCIe (the host values
    # end up the same), and the second mode is the reference's full copy-back
    modes = (("reference_eviction", False, True), ("reference_eviction_full_copy_back", False, False),
             ("frozen_host_copies", True, True))
    if args.train_modes == "reference":
        modes = modes[:1]
    if args.release_accounting == "off":
        # A/B of the eviction loop's release accounting: the budget counts the device memory that
        # save-backs in flight still hold, as it would without StagehandScheduler's hookup
        from stagehand_amd.budget import BudgetManager

        BudgetManager.count_as_released = lambda self, releasing_bytes: None
    for label, fhc, changed in modes:
        t0 = time.perf_counter()
        with torch.device("meta"):
            model = TrainDiT()
        init_train_dit_(model, args.seed, device="cuda")
        gen_s = time.perf_counter() - t0
        cfg = stagehand.StagehandConfig(pinned_pool_mb=4096, pinned_slab_mb=256, vram_high_watermark_mb=19200,
                                        vram_low_watermark_mb=14400, prefetch_window_blocks=3, max_inflight_transfers=4,
                                        nan_inf_check=False, strict_bf16=False, telemetry_enabled=True,
                                        frozen_host_copies=fhc, save_back_engine=args.save_back,
                                        save_back_changed_chunks=changed,
                                        **({} if args.run_ahead is None else {"max_run_ahead_blocks": args.run_ahead}),
                                        **({} if args.backlog_mb is None else {"save_back_backlog_mb": args.backlog_mb}))
        cfg.telemetry_file = None
        rt = stagehand.StagehandRuntime(model, cfg, block_pattern=TRAIN_BLOCK_PATTERN, dtype=torch.bfloat16,
                                        inference_mode=False)
        lora = [p for n, p in model.named_parameters() if "lora" in n]
        opt = torch.optim.SGD(lora, lr=1e-3, foreach=False)
        losses = []

        def step(i: int) -> None:
            xi = x.clone().requires_grad_()  # activations entering the blocks carry grad, as after an embedding
            rt.begin_step(i)
            with rt.managed_forward(), rt.managed_backward():
                y = model(xi, ctx, vec)
                loss = torch.nn.functional.mse_loss(y.float(), target)
                loss.backward()
            rt.end_step()
            opt.step()
            opt.zero_grad(set_to_none=True)
            losses.append(loss.detach())

        for i in range(args.train_warmup):
            step(i)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        h0, d0, l0 = rt.engine.bytes_h2d, rt.engine.bytes_d2h, rt.engine.loads
        rt.engine.host_wait_ms.clear()
        rt.scheduler.fence_kinds.clear()
        t1 = time.perf_counter()
        for i in range(args.train_steps):
            step(args.train_warmup + i)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t1
        host_waits = {k: round(v / args.train_steps, 1) for k, v in sorted(rt.engine.host_wait_ms.items())}
        fences = {k: round(v / args.train_steps, 1) for k, v in sorted(rt.scheduler.fence_kinds.items())}
        loads = rt.engine.loads - l0
        ms = wall / args.train_steps * 1e3
        h2d = (rt.engine.bytes_h2d - h0) // args.train_steps
        d2h = (rt.engine.bytes_d2h - d0) // args.train_steps
        hist = rt.telemetry.history[-args.train_steps:]
        rt.engine.start_trace()
        step(args.train_warmup + args.train_steps)
        trace = rt.engine.stop_trace()
        timeline = timeline_stats(trace, getattr(args, "pcie_peak_gbps", None))
        if trace["loads"]:
            t_first = min(l[2] for l in trace["loads"])
            timeline["load_gaps_ms_top"] = sorted(
                (round(b[2] - a[3], 2) for a, b in zip(sorted(trace["loads"], key=lambda l: l[2]),
                                                       sorted(trace["loads"], key=lambda l: l[2])[1:])),
                reverse=True)[:8]
            timeline["first_load_ms"] = round(t_first, 2)
            timeline["load_gap_causes"] = load_gap_causes(trace)
        res = {"ms_per_step": round(ms, 1), "h2d_bytes_per_step": h2d, "d2h_bytes_per_step": d2h, "timeline": timeline,
               "loads_per_step": round(loads / args.train_steps, 1),
               "host_wait_ms_per_step": host_waits, "save_back_fences_per_step": fences,
               "h2d_gbps": round(h2d / (ms * 1e-3) / 1e9, 2), "d2h_gbps": round(d2h / (ms * 1e-3) / 1e9, 2),
               "block_bytes": sum(e.size_bytes for e in rt.registry.blocks_in_order()),
               "peak_vram_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2),
               "evictions_per_step": sum(m.evictions for m in hist) / len(hist),
               "stall_ms_per_step": round(sum(m.stall_time_ms for m in hist) / len(hist), 1),
               "losses": [round(float(v), 5) for v in losses], "weights_gen_s": round(gen_s, 1),
               "steps": args.train_steps, "warmup": args.train_warmup}
        out[label] = res
        log(f"train/{label}: {res}")
        rt.shutdown()
        for e in rt.registry.blocks_in_order():
            rt.residency.get_entry(e.block_id).gpu_tensor = None
        del rt, model, opt, lora
        gc.collect()
        torch.cuda.empty_cache()
    return out


def vmm_latency_leg(args) -> dict:
    """The VMM allocator against the reference's published latencies (README.md:165-170, RTX 3090:
    ensure_resident hot path 250 ns median, ensure_resident + as_tensor 1.4 us median, eviction +
    re-map of a 1.5 GB region 4.2 ms median): the fast path timed natively and from Python, and a
    1.5 GB region mapped while the ceiling forces another one out."""
    import statistics

    import torch

    from stagehand_amd.vmm import SlabAllocator

    stream = torch.cuda.current_stream().cuda_stream
    out: dict = {}
    alloc = SlabAllocator(device=torch.cuda.current_device())
    gran = alloc.granularity()
    size = -(-(64 << 20) // gran) * gran
    slab = alloc.create_slab(size)
    reg = alloc.define_region(slab, 0, size)
    runs = [alloc.time_fast_path(slab, reg, stream, 100_000) for _ in range(5)]
    out["native_ensure_ns"] = round(statistics.median(r[0] for r in runs), 1)
    out["native_ensure_release_ns"] = round(statistics.median(r[1] for r in runs), 1)

    def median_us(fn, n=20_000):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter_ns()
            fn()
            ts.append(time.perf_counter_ns() - t0)
        return round(statistics.median(ts) / 1e3, 3)

    held = []
    out["python_ensure_us"] = median_us(lambda: held.append(alloc.ensure_resident(slab, reg, stream)))
    for h in held:
        h.release()
    held.clear()

    def ensure_tensor():
        h = alloc.ensure_resident(slab, reg, stream)
        held.append((h, h.as_tensor("bfloat16", [size // 2])))

    out["python_ensure_as_tensor_us"] = median_us(ensure_tensor)
    for h, t in held:
        del t
        h.release()
    held.clear()
    alloc.destroy_slab(slab)
    alloc.close()

    # eviction + re-map: two 1.5 GB regions under a 2 GB ceiling; each ensure_resident of the one
    # not mapped unmaps the other (its handle released, the stream idle) and maps it. An eviction
    # lowers the slab's watermark to the evicted region (vmm_src/eviction.rs:130-131), so the
    # watermark is re-opened with set_priority (vmm_backend.py activate_model) before each call
    big = -(-(1536 << 20) // gran) * gran
    alloc = SlabAllocator(device=torch.cuda.current_device(), ceiling_mb=2048)
    slab = alloc.create_slab(2 * big)
    regs = [alloc.define_region(slab, i * big, big) for i in range(2)]
    alloc.ensure_resident(slab, regs[0], stream).release()
    ts = []
    for i in range(1, 21):
        alloc.set_priority(slab, i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h = alloc.ensure_resident(slab, regs[i % 2], stream)
        ts.append((time.perf_counter() - t0) * 1e3)
        h.release()
    st = alloc.stats()
    out["evict_remap_1p5gb_ms"] = round(statistics.median(ts), 3)
    out["evict_remap_1p5gb_ms_min_max"] = [round(min(ts), 3), round(max(ts), 3)]
    out["region_bytes"] = big
    out["granularity"] = gran
    out["reference_rtx3090"] = {"ensure_resident_ns": 250, "ensure_as_tensor_us": 1.4, "evict_remap_1p5gb_ms": 4.2}
    alloc.destroy_slab(slab)
    alloc.close()
    log(f"vmm latency: {out}")
    return out


def _vmm_run(args, src: Path, ceiling_mb: int | None = None, reactivate: bool = False) -> dict:
    """Config-3 DiT served from the VMM backend: every block registered in one slab,
    filled from the sharded safetensors on first use (native loads), then resident
    in mapped device memory under the default ceiling, or under ``ceiling_mb``, which
    evicts and refills regions every step. An eviction lowers the slab's watermark to the
    evicted region (vmm_src/eviction.rs:130-131), after which the reference serves the blocks
    above it by block swap; with ``reactivate`` the model is activated again before every step
    (``VmmManager.activate_model``, which re-opens the watermark), so every step evicts and
    re-maps regions through the VMM path."""
    import gc

    import torch

    import stagehand_amd as stagehand
    from bench_workloads import DIT_BLOCK_PATTERN

    model = _dit_model()
    rt = stagehand.StagehandRuntime(model, _dit_config("file", args, False, args.file_reader), block_pattern=DIT_BLOCK_PATTERN,
                                    dtype=torch.bfloat16, inference_mode=True)
    rt.convert_registry_to_file_backed_sharded(str(src))
    handle = rt.vmm_register_model("dit", "bfloat16", str(src))
    if handle is None:
        rt.shutdown()
        return {"skipped": "VMM backend unavailable"}
    if ceiling_mb is not None:
        rt.vmm.allocator.set_vram_ceiling(int(ceiling_mb) << 20)
    img, txt, vec = _dit_inputs(args.seed)
    served = {"vmm": 0, "swap": 0}
    orig = rt._vmm_before_block

    def counted(bid, module):
        ok = orig(bid, module)
        served["vmm" if ok else "swap"] += 1
        return ok

    rt._vmm_before_block = counted

    def step(i: int):
        if reactivate:
            rt.vmm.activate_model("dit")
        rt.begin_step(i)
        with torch.no_grad(), rt.managed_forward():
            out = model(img, txt, vec)
        rt.end_step()
        return out

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step(0)
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1e3
    for i in range(args.dit_warmup):
        step(1 + i)
    torch.cuda.synchronize()
    served = {"vmm": 0, "swap": 0}
    st0 = rt.vmm.stats()
    h2d0 = rt.engine.bytes_h2d
    torch.cuda.reset_peak_memory_stats()
    t1 = time.perf_counter()
    for i in range(args.dit_steps):
        out = step(1 + args.dit_warmup + i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t1) / args.dit_steps * 1e3
    st1 = rt.vmm.stats()
    h2d = (rt.engine.bytes_h2d - h2d0) / args.dit_steps
    # fast path: ensure_resident + release of a resident region, through the Python binding
    alloc = rt.vmm.allocator
    stream = torch.cuda.current_stream().cuda_stream
    n = 2000
    fast_us = None
    try:
        t2 = time.perf_counter()
        for _ in range(n):
            alloc.ensure_resident(handle.slab_id, handle.regions[0], stream).release()
        fast_us = round((time.perf_counter() - t2) / n * 1e6, 2)
    except MemoryError:  # under a tight ceiling the region may be evicted and above the watermark
        pass
    st = rt.vmm.stats()
    res = {"file_reader": args.file_reader, "first_step_ms": round(first_ms, 1), "ms_per_step": round(ms, 2),
           "steps": args.dit_steps,
           "blocks_served_per_step": {k: v / args.dit_steps for k, v in served.items()},
           "mapped_gb": round(st["mapped_bytes"] / 1e9, 2), "vram_ceiling_gb": round(st["vram_ceiling"] / 1e9, 1),
           "granularity": st["granularity"], "maps": st["maps"], "evictions": st["evictions"],
           "ensure_release_fast_path_us": fast_us, "out_finite": bool(torch.isfinite(out.float()).all()),
           "evictions_per_step": (st1["evictions"] - st0["evictions"]) / args.dit_steps,
           "maps_per_step": (st1["maps"] - st0["maps"]) / args.dit_steps,
           "refill_bytes_per_step": int(h2d),
           "refill_gbps": round(h2d / (ms * 1e-3) / 1e9, 2),
           "reactivated_every_step": reactivate,
           # torch's allocations (block-swap buffers, activations) beside the mapped regions
           "peak_torch_allocated_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2)}
    if getattr(args, "pcie_peak_gbps", None):
        res["refill_frac_of_measured_pcie"] = round(res["refill_gbps"] / args.pcie_peak_gbps, 4)
    log(f"dit/vmm: {res}")
    rt.shutdown()
    del rt, model, out
    gc.collect()
    torch.cuda.empty_cache()
    return res


def _drop_page_cache(src: Path) -> int:
    """Writes back and drops the shards' pages from the page cache (an unprivileged
    cold start: POSIX_FADV_DONTNEED drops clean pages of the file). Returns the bytes."""
    import gc

    gc.collect()  # host views of an earlier runtime's mappings pin their pages
    total = 0
    for p in sorted(src.glob("*.safetensors")):
        fd = os.open(p, os.O_RDONLY)
        try:
            os.fsync(fd)
            os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
            total += os.fstat(fd).st_size
        finally:
            os.close(fd)
    return total


def _warm_page_cache(src: Path) -> float:
    """Reads every shard once through the page cache (a warm start for the next run); GB/s."""
    t0, total = time.perf_counter(), 0
    for p in sorted(src.glob("*.safetensors")):
        fd = os.open(p, os.O_RDONLY)
        try:
            while True:
                b = os.read(fd, 64 << 20)
                if not b:
                    break
                total += len(b)
        finally:
            os.close(fd)
    return total / (time.perf_counter() - t0) / 1e9


def _sample_read_gbps(src: Path, nbytes: int = 128 << 20) -> float:
    """Read rate of the first ``nbytes`` of the last shard: tells a cold page cache (storage
    rate) from a warm one (memory rate) after a drop."""
    p = sorted(src.glob("*.safetensors"))[-1]
    fd = os.open(p, os.O_RDONLY)
    try:
        t0 = time.perf_counter()
        done = 0
        while done < nbytes:
            b = os.pread(fd, min(16 << 20, nbytes - done), done)
            if not b:
                break
            done += len(b)
        return done / (time.perf_counter() - t0) / 1e9
    finally:
        os.close(fd)


def _first_steps(args, src: Path, reader: str, cold: bool, steps: int = 2, pinned: bool = False) -> dict:
    """A fresh runtime on the config-3 shards; wall time of each of its first steps
    (the first reads every block from the files; later ones keep part resident). With
    ``pinned`` the first load of each block fills its pinned source image and later
    loads DMA from the image."""
    import gc

    import torch

    import stagehand_amd as stagehand
    from bench_workloads import DIT_BLOCK_PATTERN

    model = _dit_model()
    rt = stagehand.StagehandRuntime(model, _dit_config("file", args, pinned, reader), block_pattern=DIT_BLOCK_PATTERN,
                                    dtype=torch.bfloat16, inference_mode=True)
    rt.convert_registry_to_file_backed_sharded(str(src))
    img, txt, vec = _dit_inputs(args.seed)
    if cold:
        file_bytes = _drop_page_cache(src)
    else:
        _warm_page_cache(src)
        file_bytes = sum(p.stat().st_size for p in src.glob("*.safetensors"))
    sample = _sample_read_gbps(src)
    torch.cuda.synchronize()
    times, sent = [], []
    for i in range(steps):
        b0 = rt.engine.bytes_h2d
        t0 = time.perf_counter()
        rt.begin_step(i)
        with torch.no_grad(), rt.managed_forward():
            out = model(img, txt, vec)
        rt.end_step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        sent.append(rt.engine.bytes_h2d - b0)
    files = rt.scheduler._weight_files.files()
    info = [f.info() for f in files]
    res = {
        "reader": reader,
        "source": "pinned source images" if pinned else "bounded pinned pool (staged)",
        "cache": "cold (dropped)" if cold else "page cache",
        "sample_read_gbps_before": round(sample, 2),
        "step_ms": [round(t * 1e3, 1) for t in times],
        "first_step_file_gbps": round(file_bytes / times[0] / 1e9, 2),
        "h2d_bytes_per_step": sent,
        "bytes_direct": sum(i["bytes_direct"] for i in info) if info else None,
        "bytes_buffered": sum(i["bytes_buffered"] for i in info) if info else None,
        "bytes_cached": sum(i["bytes_cached"] for i in info) if info else None,
        "bytes_bounced": sum(i["bytes_bounced"] for i in info) if info else None,
        "out_finite": bool(torch.isfinite(out.float()).all()),
    }
    rt.shutdown()
    for e in rt.registry.blocks_in_order():
        rt.residency.get_entry(e.block_id).gpu_tensor = None
    del rt, model, out, img, txt, vec
    gc.collect()
    torch.cuda.empty_cache()
    return res


def readers_leg(args, src: Path, main_reader: str) -> dict:
    """The weight-file readers on the config-3 shards: the first two steps of a fresh
    runtime from a cold page cache and from a warm one, and the steady-state step of
    the readers other than the main leg's."""
    import torch

    out: dict = {"file_bytes": sum(p.stat().st_size for p in src.glob("*.safetensors"))}
    # warm runs first: every shard is read through the page cache just before each
    for reader in ("mmap", "pread"):
        log(f"dit/file: reader {reader}, warm first steps")
        out[f"{reader}_warm"] = _first_steps(args, src, reader, cold=False)
    for reader in ("mmap", "pread", "direct"):
        log(f"dit/file: reader {reader}, cold first steps")
        out[f"{reader}_cold"] = _first_steps(args, src, reader, cold=True)
    log("dit/file: reader direct into pinned source images, cold first steps")
    out["direct_pinned_cold"] = _first_steps(args, src, "direct", cold=True, steps=3, pinned=True)
    for reader in ("mmap", "pread"):
        if reader == main_reader:
            continue
        log(f"dit/file: reader {reader}, steady state")
        r = _dit_run("file", args, src, None, False, reader)
        out[f"{reader}_steady"] = {k: r[k] for k in ("ms_per_step", "streamed_gbps", "pcie_bytes_per_step",
                                                     "peak_vram_gb", "timeline")}
        torch.cuda.empty_cache()
    return out


def dit_leg(kind: str, args) -> dict:
    """Streams the 19+38-block Flux-style DiT through StagehandRuntime block mode.

    kind "squareq": config 4 — int8 SquareQ slab, 6 GB VRAM cap, device dequant;
    kind "file": config 3 — bf16 sharded safetensors, 24 GB VRAM cap, prefetch window 2.
    Each source is streamed twice: through the bounded pinned pool (staged, as the
    reference does) and from pinned per-block source images.
    """
    import shutil
    import tempfile

    import torch

    from bench_workloads import write_dit_safetensors_sharded, write_dit_squareq

    model = _dit_model()
    workdir = Path(tempfile.mkdtemp(prefix=f"sh_dit_{kind}_", dir=args.workdir))
    t0 = time.perf_counter()
    if kind == "squareq":
        src = workdir / "dit.fpk"
        layers = write_dit_squareq(model, src, args.seed)
    else:
        src = workdir / "shards"
        write_dit_safetensors_sharded(model, src, args.seed)
        layers = None
    setup_s = time.perf_counter() - t0
    log(f"dit/{kind}: wrote source in {setup_s:.1f}s")
    res = {"workload": ("config4 SquareQ INT8 Flux-style DiT (19 double + 38 single blocks, hidden 3072, 11.84 B "
                        "params), 4096 image + 512 text tokens, device dequant, 6 GB VRAM cap" if kind == "squareq" else
                        "config3 bf16 Flux-style DiT (11.84 B params), sharded safetensors, 24 GB VRAM cap, prefetch window 2"),
           "source_write_s": round(setup_s, 1)}
    modes = {"staged": (False,), "pinned": (True,), "both": (False, True)}[args.dit_modes]
    reader = args.file_reader if kind == "file" else "mmap"
    for pinned in modes:
        log(f"dit/{kind}: streaming ({'pinned images' if pinned else 'staged'}, reader {reader})")
        res["pinned" if pinned else "staged"] = _dit_run(kind, args, src, layers, pinned, reader)
        torch.cuda.empty_cache()
    if kind == "file" and args.readers == "on":
        res["readers"] = readers_leg(args, src, reader)
    if kind == "file" and not args.skip_cpu:
        log("cpu baseline: the reference's config-3 block loads on a sample")
        ref3 = cpu_reference_config3_step(src)
        staged = res.get("staged") or res.get("pinned")
        if staged and staged.get("pcie_bytes_per_step"):
            # the reference evicts synchronously down to the low watermark, so it would move the
            # bytes the device path moves; its staging and H2D costs scale with them
            frac = staged["pcie_bytes_per_step"] / ref3["pcie_bytes_per_step"]
            ref3["device_traffic_fraction"] = round(frac, 4)
            ref3["ms_per_step_overlapped_at_device_traffic"] = round(ref3["ms_per_step_overlapped"] * frac, 1)
            ref3["ms_per_step_serial_at_device_traffic"] = round(ref3["ms_per_step_serial"] * frac, 1)
        res["reference_staging_path"] = ref3
    if kind == "squareq" and args.squareq_v2 == "on":
        from stagehand_amd.squareq_v2 import write_v2_slab

        v2 = workdir / "dit_v2.safetensors"
        t0 = time.perf_counter()
        write_v2_slab(str(v2), {n: {"qweight": L["qweight"], "scale": L["scale"], "bias": L["bias"]}
                                for n, L in layers.items()})  # zero points are all 0: left out
        log(f"dit/squareq: wrote the V2 slab in {time.perf_counter() - t0:.1f}s; streaming it (reader {args.file_reader})")
        r = _dit_run("squareq_v2", args, v2, layers, False, args.file_reader)
        res["v2"] = {k: r[k] for k in ("file_reader", "ms_per_step", "streamed_gbps", "pcie_bytes_per_step",
                                       "peak_vram_gb", "weight_check", "out_finite", "timeline")}
        torch.cuda.empty_cache()
    pcie = getattr(args, "pcie_peak_gbps", None)
    for m in ("staged", "pinned"):
        r = res.get(m)
        tl = r.get("timeline") if isinstance(r, dict) else None
        if pcie and tl and tl.get("compute_busy_ms"):
            # Perfect overlap: the step's copies at the measured pinned H2D rate, or its compute,
            # whichever is longer; no overlap at all: both in turn.
            copy_ms = r["pcie_bytes_per_step"] / (pcie * 1e9) * 1e3
            r["floor"] = {"copy_at_pinned_ms": round(copy_ms, 2), "compute_ms": tl["compute_busy_ms"],
                          "perfect_overlap_ms": round(max(copy_ms, tl["compute_busy_ms"]), 2),
                          "no_overlap_ms": round(copy_ms + tl["compute_busy_ms"], 2),
                          "frac_of_perfect_overlap": round(max(copy_ms, tl["compute_busy_ms"]) / r["ms_per_step"], 4)}
    best = min((res[m] for m in ("staged", "pinned") if m in res), key=lambda r: r["ms_per_step"])
    for k in ("ms_per_step", "streamed_gbps", "pcie_bytes_per_step", "block_bf16_bytes_per_step", "int8_elements",
              "scale_rows", "peak_vram_gb"):
        res[k] = best[k]
    if "floor" in best:
        res["floor"] = best["floor"]
    res["best_mode"] = best["source_mode"]
    if kind == "file" and args.vmm == "on":
        log("dit/file: served from the VMM backend")
        res["vmm"] = _vmm_run(args, src)
        log("dit/file: served from the VMM backend under a 19.2 GB ceiling (regions evicted and refilled)")
        res["vmm_tight"] = _vmm_run(args, src, ceiling_mb=19200)
        log("dit/file: VMM under a 19.2 GB ceiling, the model activated again before every step")
        res["vmm_tight_reactivated"] = _vmm_run(args, src, ceiling_mb=19200, reactivate=True)
    shutil.rmtree(workdir, ignore_errors=True)
    return res


def profile_pass(args) -> int:
    """Three launches each of the dequant and cast kernels over config 2, and of a
    plain 1 GiB byte copy through the same unpack machinery (the calibration
    kernel for HBM byte counters)."""
    import torch

    from stagehand_amd.unpack import (KIND_COPY_BYTES, UnpackPlan, dequant_i8_rowscale_bf16, make_descs,
                                      unpack_cast_f32_bf16)
    from bench_workloads import config2_descs, config2_device_inputs, config2_regions

    regions = config2_regions()
    n = sum(g.numel for g in regions)
    dst = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    plan = UnpackPlan(config2_descs(regions, "dequant"))
    src, scales = config2_device_inputs(regions, "dequant", seed=args.seed)
    for _ in range(3):
        dequant_i8_rowscale_bf16(plan, src, scales, dst)
    torch.cuda.synchronize()
    del src, scales
    cplan = UnpackPlan(config2_descs(regions, "cast"))
    csrc, _ = config2_device_inputs(regions, "cast", seed=args.seed + 1)
    for _ in range(3):
        unpack_cast_f32_bf16(cplan, csrc, dst)
    torch.cuda.synchronize()
    del csrc
    nbytes = 1 << 30
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    kplan = UnpackPlan(make_descs([(KIND_COPY_BYTES, 0, 0, 1, nbytes, 0, 0)]))
    for _ in range(3):
        kplan.run(a, b)
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": True, "dequant_algo_bytes": plan.info["algo_bytes"],
                      "cast_algo_bytes": cplan.info["algo_bytes"], "copy_bytes_each_way": nbytes}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    ap.add_argument("--skip-extras", action="store_true", help="omit cast / PCIe / D2D measurements")
    ap.add_argument("--cpu-budget-s", type=float, default=25.0)
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="config-2 legs: run the kernel this long before the warm-up and timed launches "
                         "(0 times from an idle GPU)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="only launch each kernel a few times (dequant, cast, 1 GiB copy) for counter runs")
    ap.add_argument("--dit", default="both", choices=["none", "squareq", "file", "both"],
                    help="streamed DiT legs: config 4 (squareq), config 3 (file)")
    ap.add_argument("--dit-steps", type=int, default=5)
    ap.add_argument("--dit-warmup", type=int, default=2)
    ap.add_argument("--dit-prefetch", type=int, default=2)
    ap.add_argument("--squareq-watermarks", default="3800,2800", metavar="HIGH,LOW",
                    help="config 4: VRAM watermarks in MB under its 6 GB cap")
    ap.add_argument("--workdir", default=None, help="directory for the DiT weight files (default: system temp)")
    ap.add_argument("--dit-modes", default="staged", choices=["staged", "pinned", "both"])
    ap.add_argument("--only-dit", action="store_true", help="skip the config-2 kernel legs (profiling the DiT stream)")
    ap.add_argument("--turbo", default="on", choices=["on", "off"], help="config-3 DiT through the turbo window engine")
    ap.add_argument("--train", default="on", choices=["on", "off"], help="config-5 streamed training step")
    ap.add_argument("--train-modes", default="both", choices=["both", "reference"],
                    help="config 5 with the reference's eviction (changed chunks copied back, then every byte) "
                         "and with frozen host copies, or the first only")
    ap.add_argument("--save-back", default="sdma", choices=["sdma", "stream"],
                    help="where config 5's save-back copies run (StagehandConfig.save_back_engine)")
    ap.add_argument("--vmm", default="on", choices=["on", "off"], help="config-3 DiT served from the VMM backend")
    ap.add_argument("--file-reader", default="pread", choices=["mmap", "pread", "direct"],
                    help="weight-file reader of the config-3 leg")
    ap.add_argument("--readers", default="on", choices=["on", "off"],
                    help="config-3 shards through every file reader, cold and warm page cache")
    ap.add_argument("--squareq-v2", default="on", choices=["on", "off"],
                    help="config 4 also from a SquareQ V2 slab (safetensors + manifest) through the file reader")
    ap.add_argument("--trace-markers", action="store_true",
                    help="bound the DiT legs' timed steps with marker kernels for a rocprofv3 trace")
    ap.add_argument("--trace-summary", default=None, metavar="DIR",
                    help="only summarise the copy/compute overlap of a rocprofv3 CSV trace in DIR (no GPU)")
    ap.add_argument("--trace-bytes", type=int, default=None, help="H2D bytes inside the marked window")
    ap.add_argument("--kernel-stats", default=None, metavar="DIR",
                    help="only print per-kernel dispatch statistics of a rocprofv3 kernel trace in DIR (no GPU) "
                         "over the last --steps dispatches of each kernel")
    ap.add_argument("--pmc-summary", nargs="+", default=None, metavar="DIR",
                    help="only print per-kernel medians of rocprofv3 --pmc CSVs under DIRs (no GPU)")
    ap.add_argument("--pcie-gbps", type=float, default=None, help="measured pinned H2D GB/s for --trace-summary")
    ap.add_argument("--release-accounting", default="on", choices=["on", "off"],
                    help="config 5: off counts save-back-held memory as used (A/B of the eviction loop)")
    ap.add_argument("--run-ahead", type=int, default=None,
                    help="StagehandConfig.max_run_ahead_blocks (training) and max_run_ahead_blocks_inference "
                         "(the DiT and VMM legs) (default: the config's)")
    ap.add_argument("--backlog-mb", type=int, default=None,
                    help="config 5: StagehandConfig.save_back_backlog_mb (default: the gap between the watermarks)")
    ap.add_argument("--train-steps", type=int, default=3)
    ap.add_argument("--train-warmup", type=int, default=2)
    ap.add_argument("--hw-queues", type=int, default=8,
                    help="GPU_MAX_HW_QUEUES for this process, set before HIP starts (0: leave the environment's)")
    args = ap.parse_args()
    if args.hw_queues:
        if not 1 <= args.hw_queues <= 32:
            ap.error("--hw-queues must be between 1 and 32")
        if "torch" in sys.modules:
            print("bench.py: torch was imported before --hw-queues could take effect", file=sys.stderr)
            return 2
        os.environ["GPU_MAX_HW_QUEUES"] = str(args.hw_queues)

    if args.trace_summary:
        print(json.dumps(trace_summary(Path(args.trace_summary), args.trace_bytes, args.pcie_gbps)), flush=True)
        return 0
    if args.kernel_stats:
        print(json.dumps(kernel_stats(Path(args.kernel_stats), args.steps), indent=1), flush=True)
        return 0
    if args.pmc_summary:
        print(json.dumps(pmc_summary([Path(d) for d in args.pmc_summary]), indent=1), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the streaming path runs per GPU and this build "
              "has no multi-GPU mode (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from stagehand_amd.unpack import UnpackPlan, dequant_i8_rowscale_bf16, unpack_cast_f32_bf16
    from bench_workloads import config2_descs, config2_device_inputs, config2_regions

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    if args.profile_pass:
        return profile_pass(args)
    if args.only_dit:
        args.pcie_peak_gbps = round(pinned_h2d_gbps(), 2)
        out = {"pcie": {"h2d_pinned_gbps": args.pcie_peak_gbps, "d2h_pinned_gbps": round(pinned_h2d_gbps(d2h=True), 2),
                        "duplex": duplex_gbps()}}
        if args.dit in ("squareq", "both"):
            out["dit_squareq"] = dit_leg("squareq", args)
        if args.dit in ("file", "both"):
            out["dit_file"] = dit_leg("file", args)
        if args.vmm == "on":
            out["vmm_latency"] = vmm_latency_leg(args)
        if args.turbo == "on":
            out["turbo"] = turbo_leg(args)
        if args.train == "on":
            out["train"] = train_leg(args)
        print(json.dumps(out), flush=True)
        return 0

    regions = config2_regions()
    n = sum(g.numel for g in regions)
    log(f"config 2: {len(regions)} tensors, {n} elements; generating inputs")
    plan = UnpackPlan(config2_descs(regions, "dequant"))
    src, scales = config2_device_inputs(regions, "dequant", seed=args.seed)
    dst = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    algo = plan.info["algo_bytes"]

    def step():
        dequant_i8_rowscale_bf16(plan, src, scales, dst, stream=stream)

    log(f"dequant: settle {args.settle_ms:g} ms, warmup {args.warmup}, timed {args.steps}")
    settle = settle_launches(step, args.settle_ms, stream)
    wall_ms, per = time_launches(step, args.steps, args.warmup, stream)
    avg_ms = sum(per) / len(per)
    gbps = algo / (avg_ms * 1e-3) / 1e9
    traffic = measured_traffic("sh_dequant_i8_bf16_kernel")
    result = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8->fp32->bf16",
        "data": "synthetic",
        "config": {
            "workload": "config2 SquareQ dequant: packed slab of 128 int8 tensors "
                        "(3072x3072, 3072x12288, 12288x3072, 3072x1, 1000x77 cycling), "
                        "per-row fp32 scale exp(N(-6,0.5)), bf16 RNE out",
            "elements": n,
            "rows": sum(g.rows for g in regions),
            "algo_bytes_per_step": algo,
            "parallelism": "single GPU",
            "hip_hw_queues": os.environ.get("GPU_MAX_HW_QUEUES"),
        },
        "roofline": {
            "kernel": "sh_dequant_i8_bf16_kernel",
            "bound": "hbm",
            "achieved": round(gbps, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel_ms_avg": round(avg_ms, 5),
            "kernel_ms_min": round(min(per), 5),
            **settle,
        },
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
    }

    if not args.skip_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(regions, src, scales, dst, args.cpu_budget_s)

    del src, scales
    torch.cuda.empty_cache()

    if not args.skip_extras:
        log("cast variant")
        cplan = UnpackPlan(config2_descs(regions, "cast"))
        csrc, _ = config2_device_inputs(regions, "cast", seed=args.seed + 1)

        def cstep():
            unpack_cast_f32_bf16(cplan, csrc, dst, stream=stream)

        c_settle = settle_launches(cstep, args.settle_ms, stream)
        c_wall, c_per = time_launches(cstep, args.steps, args.warmup, stream)
        c_avg = sum(c_per) / len(c_per)
        c_gbps = cplan.info["algo_bytes"] / (c_avg * 1e-3) / 1e9
        result["cast"] = {
            "kernel": "sh_cast_f32_bf16_kernel",
            "algo_bytes_per_step": cplan.info["algo_bytes"],
            "kernel_ms_avg": round(c_avg, 5),
            "gbps": round(c_gbps, 2),
            "hbm_frac": round(c_gbps / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic("sh_cast_f32_bf16_kernel"),
            **c_settle,
        }
        if not args.skip_cpu:
            log("cpu baseline: the reference's host fp32->bf16 pack")
            result["cast"]["cpu_baseline"] = cpu_cast_baseline(regions, csrc, dst, args.cpu_budget_s)
        del csrc
        torch.cuda.empty_cache()
        log("d2d copy and pinned H2D")
        result["d2d_copy_gbps"] = round(d2d_copy_gbps(), 2)
        result["copy_kernel_gbps"] = round(copy_kernel_gbps(), 2)
        result["digest_kernel"] = digest_kernel_gbps()
        result["pcie"] = {"h2d_pinned_gbps": round(pinned_h2d_gbps(), 2),
                          "d2h_pinned_gbps": round(pinned_h2d_gbps(d2h=True), 2),
                          "duplex": duplex_gbps(), "transfer_bytes": 1 << 30, "reps": 10}
        args.pcie_peak_gbps = result["pcie"]["h2d_pinned_gbps"]

    # The streamed DiTs budget VRAM with torch.cuda.memory_allocated(): release
    # every config-2 buffer first so the watermarks see only the DiT.
    del dst, plan
    if not args.skip_extras:
        del cplan
    torch.cuda.empty_cache()
    if args.dit in ("squareq", "both"):
        log("dit: config 4 (SquareQ) streaming")
        d = result["dit_squareq"] = dit_leg("squareq", args)
        if "cpu_baseline" in result:
            log("cpu baseline: the reference's config-4 block loads on a sample")
            d["reference_host_dequant_path"] = cpu_reference_config4_step(args.seed)
        if "cpu_baseline" in result and "pcie" in result:
            # The reference's config-4 path dequantises every weight on the host
            # (scheduler.py:290-300, at the CPU-baseline rate measured above) and
            # sends bf16 over PCIe; at best the two overlap.
            host_s = (d["int8_elements"] * 3 + d["scale_rows"] * 4) / (result["cpu_baseline"]["value"] * 1e9)
            h2d_s = d["block_bf16_bytes_per_step"] / (result["pcie"]["h2d_pinned_gbps"] * 1e9)
            d["reference_host_dequant_path_est"] = {
                "host_dequant_ms": round(host_s * 1e3, 1),
                "bf16_h2d_ms_at_measured_pcie": round(h2d_s * 1e3, 1),
                "ms_per_step_lower_bound": round(max(host_s, h2d_s) * 1e3, 1),
                "pcie_bytes_per_step": d["block_bf16_bytes_per_step"],
                "cores": result["cpu_baseline"]["cores"],
            }
        torch.cuda.empty_cache()
    if args.dit in ("file", "both"):
        log("dit: config 3 (file-backed bf16) streaming")
        result["dit_file"] = dit_leg("file", args)
        torch.cuda.empty_cache()
    if args.vmm == "on":
        log("vmm: allocator latencies")
        result["vmm_latency"] = vmm_latency_leg(args)
    if args.turbo == "on":
        log("turbo: config 3 DiT through the window engine")
        result["turbo"] = turbo_leg(args)
    if args.train == "on":
        log("train: config 5 streamed training step")
        result["train"] = train_leg(args)

    log(summary_line(result))
    print(json.dumps(result), flush=True)
    return 0


def summary_line(r: dict) -> str:
    """One compact line with every leg's headline figures (the driver keeps only the end of the
    output, and of the JSON line only the contract keys)."""
    def g(d, *keys, default=None):
        for k in keys:
            if not isinstance(d, dict) or k not in d:
                return default
            d = d[k]
        return d

    parts = [f"dequant {r['value']:.0f} GB/s = {r['roofline']['frac']:.3f} of HBM ({r['roofline']['kernel_ms_avg']:.4f} ms)"]
    cb = r.get("cpu_baseline")
    if cb:
        parts.append(f"cpu dequant {cb['value']} GB/s on {cb['cores']} cores, bit-exact {cb['bit_exact_vs_device']}")
    c = r.get("cast")
    if c:
        parts.append(f"cast {c['gbps']:.0f} GB/s = {c['hbm_frac']:.3f} of HBM ({c['kernel_ms_avg']:.4f} ms)")
        ccb = c.get("cpu_baseline")
        if ccb:
            parts.append(f"cpu cast {ccb['value']} GB/s, bit-exact {ccb['bit_exact_vs_device']}")
    pcie = g(r, "pcie", "h2d_pinned_gbps")
    if pcie:
        parts.append(f"pinned H2D {pcie} GB/s")
    for key, label in (("dit_squareq", "config4"), ("dit_file", "config3")):
        d = r.get(key)
        if not d:
            continue
        modes = [d[m] for m in ("staged", "pinned") if isinstance(d.get(m), dict)]
        best = next((m for m in modes if m.get("source_mode") == d.get("best_mode")), d)
        tl = best.get("timeline") or {}
        parts.append(f"{label} {d['ms_per_step']} ms/step, {d['pcie_bytes_per_step'] / 1e9:.2f} GB PCIe/step, "
                     f"{d['streamed_gbps']} GB/s = {d['streamed_gbps'] / pcie:.3f} of pinned" if pcie else
                     f"{label} {d['ms_per_step']} ms/step")
        if tl:
            parts[-1] += (f", copying {tl.get('h2d_gbps_while_copying')} GB/s, "
                          f"compute hidden {tl.get('compute_hidden_frac')}")
        fl = best.get("floor") if isinstance(best, dict) else None
        if isinstance(fl, dict):
            parts[-1] += (f", perfect-overlap floor {fl['perfect_overlap_ms']} ms (copies {fl['copy_at_pinned_ms']}, "
                          f"compute {fl['compute_ms']}) = {fl['frac_of_perfect_overlap']:.3f} of it")
        wc = best.get("weight_check") if isinstance(best, dict) else None
        if isinstance(wc, dict) and "resident_layers_checked" in wc:
            parts[-1] += f", weights bit-exact {wc['bit_exact']} on {wc['resident_layers_checked']} resident layers"
        if isinstance(wc, dict) and "resident_blocks_checked" in wc:
            parts[-1] += (f", weights bit-exact {wc['bit_exact']} on {wc['resident_blocks_checked']} resident blocks "
                          f"({wc['bytes_checked'] / 1e9:.2f} GB)")
        ref = d.get("reference_host_dequant_path")
        if ref:
            parts.append(f"{label} reference host path {ref['ms_per_step']} ms/step on {ref['cores']} cores")
    vmm = g(r, "dit_file", "vmm")
    if isinstance(vmm, dict) and "ms_per_step" in vmm:
        parts.append(f"vmm {vmm['ms_per_step']} ms/step")
    vt = g(r, "dit_file", "vmm_tight")
    if isinstance(vt, dict) and "ms_per_step" in vt:
        parts.append(f"vmm 19.2 GB ceiling {vt['ms_per_step']} ms/step, {vt['evictions_per_step']} evictions/step, "
                     f"refill {vt['refill_gbps']} GB/s")
    vr = g(r, "dit_file", "vmm_tight_reactivated")
    if isinstance(vr, dict) and "ms_per_step" in vr:
        bs = vr.get("blocks_served_per_step") or {}
        parts.append(f"vmm 19.2 GB re-activated {vr['ms_per_step']} ms/step, {vr['evictions_per_step']} evictions + "
                     f"{vr['maps_per_step']} maps/step, {bs.get('vmm')} blocks from VMM, {bs.get('swap')} swapped")
    vl = r.get("vmm_latency")
    if isinstance(vl, dict) and "native_ensure_ns" in vl:
        parts.append(f"vmm ensure {vl['native_ensure_ns']} ns native, {vl['python_ensure_us']} us python, "
                     f"+as_tensor {vl['python_ensure_as_tensor_us']} us, evict+remap 1.5 GB {vl['evict_remap_1p5gb_ms']} ms")
    t = r.get("turbo")
    if t:
        for mode in ("engine_layout", "reference_layout", "reference_layout_full_write_back"):
            if isinstance(t.get(mode), dict):
                parts.append(f"turbo/{mode} {t[mode]['ms_per_step']} ms/step, pcie {t[mode].get('pcie_frac')}")
    tr = r.get("train")
    if tr:
        for mode, d in tr.items():
            if isinstance(d, dict) and "ms_per_step" in d:
                d2h = d.get("d2h_bytes_per_step")
                parts.append(f"train/{mode} {d['ms_per_step']} ms/step"
                             + (f", D2H {d2h / 1e9:.2f} GB/step" if isinstance(d2h, (int, float)) else ""))
    return "summary: " + " | ".join(parts)


if __name__ == "__main__":
    sys.exit(main())
