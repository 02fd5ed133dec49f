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
