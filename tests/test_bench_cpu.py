"""The bench's reporting helpers, on the CPU: the rocprofv3 trace summary and the summary line.

``bench.py --trace-summary`` turns rocprofv3 kernel and memory-copy CSVs into the copy/compute
overlap of the marked steps; a synthetic trace with known intervals pins its arithmetic.
"""
from __future__ import annotations

import csv

import pytest

import bench

K_FIELDS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
            "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
C_FIELDS = ["Kind", "Direction", "Stream_Id", "Source_Agent_Id", "Destination_Agent_Id", "Correlation_Id",
            "Start_Timestamp", "End_Timestamp"]


def _write(tmp_path, kernels, copies):
    with open(tmp_path / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, K_FIELDS)
        w.writeheader()
        for i, (name, a, b) in enumerate(kernels):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Dispatch_Id": i, "Start_Timestamp": a,
                        "End_Timestamp": b})
    with open(tmp_path / "run_memory_copy_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, C_FIELDS)
        w.writeheader()
        for d, a, b in copies:
            w.writerow({"Kind": "MEMORY_COPY", "Direction": f"MEMORY_COPY_{d}", "Start_Timestamp": a,
                        "End_Timestamp": b})


def test_trace_summary_overlap_arithmetic(tmp_path):
    ms = 1_000_000  # timestamps in ns
    kernels = [
        ("sh_put_descs_kernel", 0, 1 * ms),          # marker: the window starts at 1 ms
        ("Cijk_gemm", 2 * ms, 6 * ms),               # compute 4 ms, 2 ms under a copy
        ("attn_fwd", 5 * ms, 9 * ms),                # compute overlapping the gemm: union 2..9 = 7 ms
        ("sh_dequant_i8_bf16_kernel", 9 * ms, 10 * ms),  # unpack, not compute
        ("elementwise", 30 * ms, 31 * ms),           # after the window: ignored
        ("sh_put_descs_kernel", 20 * ms, 21 * ms),   # marker: the window ends at 20 ms
    ]
    copies = [
        ("HOST_TO_DEVICE", 0, 4 * ms),               # clipped to 1..4 = 3 ms
        ("HOST_TO_DEVICE", 8 * ms, 12 * ms),         # 4 ms, 1 ms under compute (8..9)
        ("DEVICE_TO_HOST", 12 * ms, 13 * ms),
        ("HOST_TO_DEVICE", 25 * ms, 26 * ms),        # outside
    ]
    _write(tmp_path, kernels, copies)
    out = bench.trace_summary(tmp_path, h2d_bytes=7 * 10**8, pcie_gbps=200.0)
    assert out["window_ms"] == 19.0
    assert out["h2d_copies"] == 2 and out["h2d_busy_ms"] == 7.0
    assert out["compute_kernels"] == 2 and out["compute_busy_ms"] == 7.0
    assert out["unpack_kernels"] == 1 and out["unpack_busy_ms"] == 1.0
    assert out["d2h_busy_ms"] == 1.0
    assert out["h2d_compute_overlap_ms"] == 3.0  # 2..4 and 8..9
    assert out["compute_hidden_frac"] == pytest.approx(3 / 7, abs=1e-4)
    assert out["h2d_gbps_while_copying"] == 100.0  # 0.7 GB in 7 ms
    assert out["frac_of_measured_pinned_pcie_while_copying"] == 0.5


def test_trace_summary_from_a_kernel_trace_alone(tmp_path):
    """Without a memory-copy trace: compute busy, its idle stretches and the blocks' arrivals (the
    unpack kernels' starts) in the marked window."""
    ms = 1_000_000
    kernels = [
        ("sh_put_descs_kernel", 0, 1 * ms),                  # the window starts at 1 ms
        ("sh_unpack_mixed_kernel", 1 * ms, 2 * ms),          # block 1 lands at 1 ms
        ("Cijk_gemm", 2 * ms, 5 * ms),
        ("sh_unpack_mixed_kernel", 4 * ms, 5 * ms),          # block 2 at 4 ms
        ("attn_fwd", 5 * ms, 7 * ms),                        # compute 2..7, then idle 7..9
        ("sh_dequant_i8_bf16_kernel", 8 * ms, 9 * ms),       # block 3 at 8 ms
        ("elementwise", 9 * ms, 10 * ms),
        ("sh_put_descs_kernel", 11 * ms, 12 * ms),           # the window ends at 11 ms
    ]
    with open(tmp_path / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, K_FIELDS)
        w.writeheader()
        for i, (name, a, b) in enumerate(kernels):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Dispatch_Id": i, "Start_Timestamp": a,
                        "End_Timestamp": b})
    out = bench.trace_summary(tmp_path, h2d_bytes=10**9, pcie_gbps=200.0)
    assert out["window_ms"] == 10.0
    assert out["compute_kernels"] == 3 and out["compute_busy_ms"] == 6.0
    assert out["compute_busy_frac"] == 0.6
    assert out["compute_idle_top_ms"] == [2.0]
    assert out["unpack_kernels"] == 3 and out["unpack_busy_ms"] == 3.0
    assert out["arrival_interval_ms"] == {"median": 3.5, "min": 3.0, "max": 4.0}
    assert out["h2d_gbps_over_window"] == 100.0
    assert out["frac_of_measured_pinned_pcie_over_window"] == 0.5
    assert "h2d_busy_ms" not in out


def test_trace_summary_needs_two_markers(tmp_path):
    _write(tmp_path, [("sh_put_descs_kernel", 0, 1)], [("HOST_TO_DEVICE", 0, 1)])
    with pytest.raises(ValueError):
        bench.trace_summary(tmp_path, None, None)


def test_summary_line_names_every_leg():
    r = {"value": 6200.0, "roofline": {"frac": 0.775, "kernel_ms_avg": 1.07},
         "cpu_baseline": {"value": 4.1, "cores": 16, "bit_exact_vs_device": True},
         "cast": {"gbps": 6000.0, "hbm_frac": 0.75, "kernel_ms_avg": 2.2,
                  "cpu_baseline": {"value": 3.0, "bit_exact_vs_device": True}},
         "pcie": {"h2d_pinned_gbps": 57.0},
         "dit_squareq": {"ms_per_step": 212.0, "pcie_bytes_per_step": 11.85e9, "streamed_gbps": 55.9,
                         "best_mode": "staged", "staged": {"source_mode": "staged",
                                                           "timeline": {"h2d_gbps_while_copying": 55.6,
                                                                        "compute_hidden_frac": 0.98}}},
         "train": {"reference_eviction": {"ms_per_step": 1000.0}}}
    line = bench.summary_line(r)
    for want in ("dequant 6200 GB/s", "cast 6000 GB/s", "cpu cast 3.0", "config4 212.0 ms/step",
                 "compute hidden 0.98", "train/reference_eviction 1000.0"):
        assert want in line, (want, line)
    assert "\n" not in line


def test_summary_line_reports_config3_floor_and_weight_check():
    r = {"value": 6200.0, "roofline": {"frac": 0.775, "kernel_ms_avg": 1.07}, "pcie": {"h2d_pinned_gbps": 57.0},
         "dit_file": {"ms_per_step": 188.0, "pcie_bytes_per_step": 7.76e9, "streamed_gbps": 41.3,
                      "best_mode": "staged",
                      "staged": {"source_mode": "staged", "timeline": {"h2d_gbps_while_copying": 54.5,
                                                                        "compute_hidden_frac": 0.58},
                                 "floor": {"copy_at_pinned_ms": 135.5, "compute_ms": 122.1, "perfect_overlap_ms": 135.5,
                                           "no_overlap_ms": 257.6, "frac_of_perfect_overlap": 0.7207},
                                 "weight_check": {"resident_blocks_checked": 30, "file_params_checked": 300,
                                                  "module_params": 60, "bytes_checked": 15.1e9, "bit_exact": True}}}}
    line = bench.summary_line(r)
    for want in ("config3 188.0 ms/step", "perfect-overlap floor 135.5 ms", "= 0.721 of it",
                 "weights bit-exact True on 30 resident blocks (15.10 GB)"):
        assert want in line, (want, line)


def test_file_weight_check_compares_resident_buffers_with_the_shards(tmp_path):
    """The bench's config-3 weight check on a tiny sharded model streamed on the host path: every
    file-backed parameter of every resident block matches its shard bytes, and one flipped byte in
    a resident buffer is caught."""
    import json

    import torch
    from safetensors.torch import save_file

    import stagehand_amd as stagehand
    from stagehand_amd.config import StagehandConfig
    from tests.streaming_models import TinyStack, init_

    if torch.cuda.is_available():
        pytest.skip("the host block path runs where there is no GPU")
    model = init_(TinyStack(n=3, hidden=32, mlp=2)).to(torch.bfloat16)
    shards = tmp_path / "shards"
    shards.mkdir()
    weight_map = {}
    for bi, blk in enumerate(model.blocks):
        tensors = {f"blocks.{bi}.{n}": p.detach().clone() for n, p in blk.named_parameters()}
        save_file(tensors, str(shards / f"b{bi}.safetensors"))
        weight_map.update({k: f"b{bi}.safetensors" for k in tensors})
    (shards / "diffusion_pytorch_model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    for p in model.parameters():
        p.requires_grad_(False)
    cfg = StagehandConfig(pinned_pool_mb=8, pinned_slab_mb=1, vram_high_watermark_mb=200000,
                          vram_low_watermark_mb=100000, prefetch_window_blocks=1, telemetry_enabled=False,
                          nan_inf_check=False, strict_bf16=False)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_file_backed_sharded(str(shards)) > 0
    rt.begin_step(0)
    with torch.no_grad(), rt.managed_forward():
        model(torch.randn(2, 32).to(torch.bfloat16))
    rt.end_step()
    check = bench._file_weight_check(rt)
    assert check["bit_exact"] is True and check["resident_blocks_checked"] == 3
    assert check["file_params_checked"] > 0 and check["bytes_checked"] > 0
    entry = rt.registry.get("blocks.1")
    filed = {f.param_name for f in entry.file_param_specs}
    off = next(o for name, _s, _d, o, n in entry.param_layout if name in filed and n > 2)
    buf = rt.residency.get_entry("blocks.1").gpu_tensor
    buf.view(torch.uint8)[off + 3] ^= 0x40
    assert bench._file_weight_check(rt)["bit_exact"] is False
    rt.shutdown()
