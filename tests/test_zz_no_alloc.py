"""The allocation-free unpack entry point (``sh_unpack_noalloc``) against the plan-based one.

``sh_unpack_noalloc`` keeps the launch table and tile map in the library's static per-GPU
scratch instead of device memory ``sh_plan_create`` allocates; the unpack kernels are the same.
Its output must equal ``sh_unpack`` on the same descriptors and inputs byte for byte. Two calls
in a row share the scratch: the first is config 2's full dequant (128 descriptors, 270k tiles),
the second a smaller mixed table whose table and tile map only partly overwrite the first's.
Calls issued back to back on two streams are ordered on the device (each waits for the previous
call's kernels before it writes the shared table), so both outputs stay exact. Limits are refused
with SH_ERR_INVALID before anything is launched.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bench_workloads import config2_descs, config2_device_inputs, config2_regions
from oracle import squareq as oq
from stagehand_amd import _native
from stagehand_amd.unpack import (
    KIND_BF16_F32,
    KIND_COPY_BYTES,
    KIND_F32_BF16,
    KIND_I8_ROWSCALE_BF16,
    KIND_I8_ROWSCALE_F32,
    KIND_ZERO_BYTES,
    UnpackPlan,
    make_descs,
    unpack_noalloc,
)

pytestmark = pytest.mark.gpu


def _mixed_case(seed: int):
    """A mixed table of 47 regions (two chunks of descriptor arguments), unaligned int8 sources,
    padded rows and zero points."""
    rng = np.random.default_rng(seed)
    rows = []
    src_parts, off = [], 5
    dst_off, scale_off = 0, 0

    def add_src(a: np.ndarray, align: int = 1) -> int:
        nonlocal off
        off = (off + align - 1) // align * align
        src_parts.append((off, a))
        at = off
        off += a.nbytes
        return at

    q = rng.integers(-127, 128, (300, 80), dtype=np.int8)
    rows.append((KIND_I8_ROWSCALE_BF16, add_src(q), dst_off, 300, 77, 80, scale_off))
    dst_off += 300 * 77 * 2
    scale_off += 300
    q2 = rng.integers(-127, 128, (64, 33), dtype=np.int8)
    rows.append((KIND_I8_ROWSCALE_F32, add_src(q2), dst_off, 64, 33, 0, scale_off))
    dst_off += 64 * 33 * 4
    scale_off += 64
    f = (rng.standard_normal(1000) * 0.02).astype(np.float32)
    rows.append((KIND_F32_BF16, add_src(f, 4), dst_off, 1, 1000, 0, 0))
    dst_off += 2000
    b = rng.integers(0, 1 << 16, 555, dtype=np.uint16)
    b[(b & 0x7F80) == 0x7F80] = 0x3F80  # no NaN/inf patterns: plain values
    rows.append((KIND_BF16_F32, add_src(b, 2), dst_off, 1, 555, 0, 0))
    dst_off += 555 * 4
    raw = rng.integers(0, 256, 12345, dtype=np.uint8)
    rows.append((KIND_COPY_BYTES, add_src(raw), dst_off, 1, 12345, 0, 0))
    dst_off += 12345
    rows.append((KIND_ZERO_BYTES, 0, dst_off, 1, 777, 0, 0))
    dst_off += 777
    dst_off = (dst_off + 1) // 2 * 2
    for _ in range(41):
        qs = rng.integers(-127, 128, (10, 17), dtype=np.int8)
        rows.append((KIND_I8_ROWSCALE_BF16, add_src(qs), dst_off, 10, 17, 0, scale_off))
        dst_off += 10 * 17 * 2
        scale_off += 10
    slab = np.zeros(off + 64, dtype=np.uint8)
    for o, a in src_parts:
        slab[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    scales = np.exp(rng.normal(-6.0, 0.5, scale_off)).astype(np.float32)
    zps = rng.normal(0.0, 2.0, scale_off).astype(np.float32)
    return make_descs(rows), slab, scales, zps, dst_off, (q, scales[:300], zps[:300])


def _both(descs, src, scales, zps, dst_bytes):
    """Runs the plan-based entry point and the allocation-free one into 0xA5-filled buffers."""
    want = torch.full((dst_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
    got = torch.full((dst_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
    plan = UnpackPlan(descs)
    plan.run(src, want, scales, zps)
    plan.close()
    unpack_noalloc(descs, src, got, scales, zps)
    torch.cuda.synchronize()
    return want, got


def test_noalloc_matches_plan_entry_point_two_calls_in_a_row():
    # call 1: config 2's full dequant slab
    regions = config2_regions()
    descs = config2_descs(regions, "dequant")
    src, scales = config2_device_inputs(regions, "dequant", seed=3)
    n = sum(g.numel for g in regions)
    want, got = _both(descs, src, scales, None, 2 * n)
    assert torch.equal(want, got), "config-2 dequant: sh_unpack_noalloc differs from sh_unpack"
    del want, got, src, scales
    torch.cuda.empty_cache()

    # call 2: a smaller mixed table, into the scratch the first call left behind
    descs2, slab, sc, zp, dst_bytes, (q, s300, z300) = _mixed_case(seed=4)
    assert len(descs2) > 32  # more than one chunk of descriptor arguments
    want, got = _both(descs2, torch.from_numpy(slab).cuda(), torch.from_numpy(sc).cuda(),
                      torch.from_numpy(zp).cuda(), dst_bytes + 16)
    assert torch.equal(want, got), "mixed table: sh_unpack_noalloc differs from sh_unpack"
    first = got[:300 * 77 * 2].cpu().numpy().view(np.uint16).reshape(300, 77)
    assert np.array_equal(first, oq.dequant_rows(q, s300, z300, 300, 77))  # and both equal the oracle
    assert (got[dst_bytes:].cpu().numpy() == 0xA5).all()  # nothing written past the table

    # call 3: the first table again, after the smaller one: same bytes as call 2
    again = torch.full((dst_bytes + 16,), 0xA5, dtype=torch.uint8, device="cuda")
    unpack_noalloc(descs2, torch.from_numpy(slab).cuda(), again, torch.from_numpy(sc).cuda(),
                   torch.from_numpy(zp).cuda())
    torch.cuda.synchronize()
    assert torch.equal(again, want)


def test_noalloc_calls_on_two_streams_do_not_corrupt_each_other():
    """A long call (config 2's full dequant, about 1 ms of kernels) on one stream and, issued right
    after it, a short call with another table on a second stream, then the long one again on the
    second stream and a short one on the first. Without ordering, the second call's table writes
    would land while the first call's unpack still reads the table."""
    regions = config2_regions()
    descs_a = config2_descs(regions, "dequant")
    src_a, scales_a = config2_device_inputs(regions, "dequant", seed=5)
    bytes_a = 2 * sum(g.numel for g in regions)
    descs_b, slab, sc, zp, bytes_b, _ = _mixed_case(seed=6)
    src_b, sc_b, zp_b = torch.from_numpy(slab).cuda(), torch.from_numpy(sc).cuda(), torch.from_numpy(zp).cuda()

    want_a = torch.full((bytes_a,), 0xA5, dtype=torch.uint8, device="cuda")
    want_b = torch.full((bytes_b,), 0xA5, dtype=torch.uint8, device="cuda")
    for descs, src, sc_, zp_, want in ((descs_a, src_a, scales_a, None, want_a), (descs_b, src_b, sc_b, zp_b, want_b)):
        plan = UnpackPlan(descs)
        plan.run(src, want, sc_, zp_)
        plan.close()
    got_a1 = torch.full_like(want_a, 0xA5)
    got_b1 = torch.full_like(want_b, 0xA5)
    got_a2 = torch.full_like(want_a, 0xA5)
    got_b2 = torch.full_like(want_b, 0xA5)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    unpack_noalloc(descs_a, src_a, got_a1, scales_a, None, stream=s1)
    unpack_noalloc(descs_b, src_b, got_b1, sc_b, zp_b, stream=s2)
    unpack_noalloc(descs_a, src_a, got_a2, scales_a, None, stream=s2)
    unpack_noalloc(descs_b, src_b, got_b2, sc_b, zp_b, stream=s1)
    torch.cuda.synchronize()
    assert torch.equal(got_a1, want_a), "first long call corrupted by the call on the other stream"
    assert torch.equal(got_b1, want_b)
    assert torch.equal(got_a2, want_a)
    assert torch.equal(got_b2, want_b)


def test_noalloc_refuses_tables_beyond_its_scratch():
    lib = _native.lib()
    # more tiles than the scratch's tile map holds (fp32 cast tiles: 2048 elements)
    per_tile = 2048
    too_many_tiles = make_descs([(KIND_F32_BF16, 0, 0, _native_max_tiles() + 1, per_tile, 0, 0)])
    st = lib.sh_unpack_noalloc(too_many_tiles.ctypes.data, 1, None, 0, None, None, 0, None, 0, None)
    assert st == _native.SH_ERR_INVALID and b"tiles" in lib.sh_last_error()
    # more descriptors than the scratch's table holds
    many = make_descs([(KIND_ZERO_BYTES, 0, 16 * i, 1, 16, 0, 0) for i in range(2049)])
    st = lib.sh_unpack_noalloc(many.ctypes.data, len(many), None, 0, None, None, 0, None, 0, None)
    assert st == _native.SH_ERR_INVALID and b"descriptors" in lib.sh_last_error()
    # a too-small destination is refused as by sh_unpack
    small = make_descs([(KIND_ZERO_BYTES, 0, 0, 1, 4096, 0, 0)])
    dst = torch.zeros(100, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        unpack_noalloc(small, None, dst)


def _native_max_tiles() -> int:
    return 2064384
