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


def pinned_h2d_gbps(reps: int = 10, nbytes: int = 1 << 30) -> float:
    import torch

    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    host.fill_(1)
    dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        dev.copy_(host, non_blocking=True)
    stream.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(reps):
            dev.copy_(host, non_blocking=True)
    t1.record(stream)
    stream.synchronize()
    return reps * nbytes / (t0.elapsed_time(t1) * 1e-3) / 1e9


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


def cpu_baseline(regions, src, scales, dst, budget_s: float) -> dict:
    """The reference's host dequant (torch CPU ops) on a bounded sample; bit-checked against dst."""
    import torch

    from oracle.torch_ref import host_dequant_into

    threads = min(os.cpu_count() or 1, 16)
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
    host_dequant_into(slab, work)  # warm
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        host_dequant_into(slab, work)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
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
                   f"median of {len(times)} runs"),
        "ms_per_sample": round(med * 1e3, 2),
        "bit_exact_vs_device": bit_exact,
    }


def profile_pass(args) -> int:
    """Three launches each of the dequant and cast kernels over config 2, and of a
    plain 1 GiB byte copy through the same unpack machinery (the calibration
    kernel for HBM byte counters)."""
    import torch

    from stagehand_amd.unpack import (KIND_COPY_BYTES, UnpackPlan, dequant_i8_rowscale_bf16, make_descs,
                                      unpack_cast_f32_bf16)
    from stagehand_amd.workloads import config2_descs, config2_device_inputs, config2_regions

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
    ap.add_argument("--profile-pass", action="store_true",
                    help="only launch each kernel a few times (dequant, cast, 1 GiB copy) for counter runs")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the streaming path runs per GPU and this build "
              "has no multi-GPU mode (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from stagehand_amd.unpack import UnpackPlan, dequant_i8_rowscale_bf16, unpack_cast_f32_bf16
    from stagehand_amd.workloads import config2_descs, config2_device_inputs, config2_regions

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    if args.profile_pass:
        return profile_pass(args)

    regions = config2_regions()
    n = sum(g.numel for g in regions)
    log(f"config 2: {len(regions)} tensors, {n} elements; generating inputs")
    plan = UnpackPlan(config2_descs(regions, "dequant"))
    src, scales = config2_device_inputs(regions, "dequant", seed=args.seed)
    dst = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    algo = plan.info["algo_bytes"]

    def step():
        dequant_i8_rowscale_bf16(plan, src, scales, dst, stream=stream)

    log(f"dequant: warmup {args.warmup}, timed {args.steps}")
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
        }
        del csrc
        torch.cuda.empty_cache()
        log("d2d copy and pinned H2D")
        result["d2d_copy_gbps"] = round(d2d_copy_gbps(), 2)
        result["pcie"] = {"h2d_pinned_gbps": round(pinned_h2d_gbps(), 2), "transfer_bytes": 1 << 30, "reps": 10}

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
