"""Parity of the HIP unpack kernels (through the C ABI) with the CPU oracle.

Bar: bit-exact bf16 / fp32 output. Small cases are compared with
oracle/squareq.py and the golden fixtures; the full config-2 slab (2.2 G
elements) is compared bit for bit with torch's device ops of the same
expression — itself checked against the oracle on sampled rows in the same
test — and the fp32→bf16 conversion is checked on all 2^32 bit patterns.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import squareq as oq
from stagehand_amd.unpack import (
    KIND_BF16_F32,
    KIND_COPY_BYTES,
    KIND_F32_BF16,
    KIND_I8_ROWSCALE_BF16,
    KIND_I8_ROWSCALE_F32,
    KIND_ZERO_BYTES,
    UnpackPlan,
    dequant_i8_rowscale_bf16,
    make_descs,
    unpack_cast_f32_bf16,
)
from bench_workloads import config2_descs, config2_device_inputs, config2_regions

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy().view(np.uint16)


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _pack(arrays: list[np.ndarray], start: int = 0, align: int = 1) -> tuple[np.ndarray, list[int]]:
    """Packs raw bytes of arrays back to back from byte `start`; returns (uint8 slab, offsets)."""
    offs, pos = [], start
    for a in arrays:
        pos = (pos + align - 1) // align * align
        offs.append(pos)
        pos += a.nbytes
    slab = np.zeros(pos + 64, dtype=np.uint8)
    for a, o in zip(arrays, offs):
        slab[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    return slab, offs


def test_golden_rows_through_kernel():
    z = _golden("squareq_rows.npz")
    qs = [z[f"q{i}"] for i in range(5)]
    slab, offs = _pack(qs, start=3)
    scales = np.concatenate([z[f"s{i}"] for i in range(5)])
    rows_off = np.cumsum([0] + [q.shape[0] for q in qs])
    dst_off = np.cumsum([0] + [q.size * 2 for q in qs])
    descs = make_descs((KIND_I8_ROWSCALE_BF16, offs[i], int(dst_off[i]), q.shape[0], q.shape[1], 0, int(rows_off[i]))
                       for i, q in enumerate(qs))
    plan = UnpackPlan(descs)
    dst = torch.empty(int(dst_off[-1]) // 2, dtype=torch.bfloat16, device="cuda")
    dequant_i8_rowscale_bf16(plan, _dev(slab), _dev(scales), dst)
    torch.cuda.synchronize()
    got = _u16(dst)
    for i in range(5):
        np.testing.assert_array_equal(got[dst_off[i] // 2:dst_off[i + 1] // 2], z[f"out{i}"].reshape(-1))

    # special scales and zero points: inf/nan/denormal/overflow, with zero points
    qe, se, ze = z["q_edge"], z["s_edge"], z["z_edge"]
    for kind, want, width in ((KIND_I8_ROWSCALE_BF16, z["out_edge"], 2), (KIND_I8_ROWSCALE_F32, z["outf32_edge"], 4)):
        plan = UnpackPlan(make_descs([(kind, 0, 0, qe.shape[0], qe.shape[1], 0, 0)]))
        dst = torch.empty(qe.size * width, dtype=torch.uint8, device="cuda")
        plan.run(_dev(qe), dst, _dev(se), _dev(ze))
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        if width == 2:
            np.testing.assert_array_equal(got.view(np.uint16).reshape(qe.shape), want)
        else:
            np.testing.assert_array_equal(got.view(np.uint32).reshape(qe.shape), want.view(np.uint32))


def test_reference_known_answer_through_kernel():
    """tests/test_scheduler.py:307-373 of the reference, through the device path (bf16 and fp32)."""
    z = _golden("squareq_known_answer.npz")
    q = z["qweight"]
    for kind, width in ((KIND_I8_ROWSCALE_BF16, 2), (KIND_I8_ROWSCALE_F32, 4)):
        plan = UnpackPlan(make_descs([(kind, 0, 0, 8, 8, 0, 0), (KIND_F32_BF16 if width == 2 else KIND_COPY_BYTES,
                                                                   64, 64 * width, 1, 8 if width == 2 else 32, 0, 0)]))
        src = np.zeros(64 + 32, np.uint8)
        src[:64] = q.view(np.uint8).reshape(-1)
        src[64:96] = z["bias"].view(np.uint8)
        dst = torch.empty(72 * width, dtype=torch.uint8, device="cuda")
        plan.run(_dev(src), dst, _dev(z["scale"]), _dev(z["zero_point"]))
        torch.cuda.synchronize()
        out = dst.cpu().numpy()
        if width == 2:
            np.testing.assert_array_equal(out[:128].view(np.uint16), z["weight_bf16_bits"].reshape(-1))
            np.testing.assert_array_equal(out[128:].view(np.uint16), z["bias_bf16_bits"])
        else:
            np.testing.assert_array_equal(out[:256].view(np.float32), q.astype(np.float32).reshape(-1))
            np.testing.assert_array_equal(out[256:].view(np.float32), z["bias"])


CASES = [
    # rows, cols, ld, src_misalign, dst_misalign(bytes, even), zp
    (64, 3072, 3072, 0, 0, False),
    (37, 3072, 3072, 8, 0, False),
    (5, 12288, 12288, 3, 2, True),
    (3072, 1, 1, 0, 0, False),
    (1000, 77, 77, 8, 0, False),
    (33, 77, 77, 5, 6, True),
    (17, 16, 16, 1, 2, False),
    (9, 48, 64, 2, 0, True),    # padded source rows (padded_in > in)
    (11, 100, 100, 0, 4, False),
    (2, 7, 7, 0, 0, True),
    (1, 40000, 40000, 7, 10, False),
    (3, 4097, 4097, 1, 2, False),
]


@pytest.mark.parametrize("rows,cols,ld,smis,dmis,use_zp", CASES)
@pytest.mark.parametrize("out", ["bfloat16", "float32"])
def test_dequant_random_shapes_match_oracle(rows, cols, ld, smis, dmis, use_zp, out):
    rng = np.random.default_rng(rows * 7919 + cols * 31 + ld)
    q = rng.integers(-128, 128, (rows, ld), dtype=np.int8)
    s = np.exp(rng.normal(-6.0, 0.5, rows + 3)).astype(np.float32)
    s[::7] = rng.normal(0, 1, s[::7].size).astype(np.float32)  # some negative / large scales
    zp = rng.normal(0, 3, rows + 3).astype(np.float32) if use_zp else None
    width = 2 if out == "bfloat16" else 4
    kind = KIND_I8_ROWSCALE_BF16 if out == "bfloat16" else KIND_I8_ROWSCALE_F32
    src = np.zeros(smis + q.size + 64, np.uint8)
    src[smis:smis + q.size] = q.view(np.uint8).reshape(-1)
    plan = UnpackPlan(make_descs([(kind, smis, dmis, rows, cols, ld, 3)]))
    dst = torch.full((dmis + rows * cols * width + 32,), 0xAB, dtype=torch.uint8, device="cuda")
    plan.run(_dev(src), dst, _dev(s), _dev(zp) if zp is not None else None)
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    want = oq.dequant_rows(q, s[3:], zp[3:] if zp is not None else None, rows, cols, out=out)
    body = got[dmis:dmis + rows * cols * width]
    if width == 2:
        np.testing.assert_array_equal(body.view(np.uint16).reshape(rows, cols), want)
    else:
        np.testing.assert_array_equal(body.view(np.uint32).reshape(rows, cols), want.view(np.uint32))
    assert (got[:dmis] == 0xAB).all() and (got[dmis + rows * cols * width:] == 0xAB).all(), "wrote outside its region"


def test_mixed_plan_all_kinds_match_oracle():
    rng = np.random.default_rng(11)
    w = rng.integers(-127, 128, (24, 80), dtype=np.int8)
    s = np.exp(rng.normal(-6, 0.5, 24)).astype(np.float32)
    b32 = rng.normal(0, 1, 24).astype(np.float32)
    nrm = rng.normal(1, 0.1, 333).astype(np.float32)
    bf = oq.cast_f32_bf16(rng.normal(0, 1, 50).astype(np.float32))
    raw = rng.integers(0, 256, 1001, dtype=np.uint8)
    src, (o_w, o_b, o_n, o_bf, o_raw) = _pack([w, b32, nrm, bf, raw], start=5)
    # destination: fp32 runtime regions and bf16 regions interleaved at odd-but-even offsets
    layout = [("w", 24 * 80 * 2), ("b", 24 * 2), ("n", 333 * 2), ("bf", 50 * 4), ("raw", 1001), ("z", 77)]
    doff, pos = {}, 2
    for name, nb in layout:
        doff[name] = pos
        pos += nb
    descs = make_descs([
        (KIND_I8_ROWSCALE_BF16, o_w, doff["w"], 24, 80, 0, 0),
        (KIND_F32_BF16, o_b, doff["b"], 1, 24, 0, 0),
        (KIND_F32_BF16, o_n, doff["n"], 1, 333, 0, 0),
        (KIND_BF16_F32, o_bf, doff["bf"], 1, 50, 0, 0),
        (KIND_COPY_BYTES, o_raw, doff["raw"], 1, 1001, 0, 0),
        (KIND_ZERO_BYTES, 0, doff["z"], 1, 77, 0, 0),
    ])
    plan = UnpackPlan(descs)
    dst = torch.full((pos + 16,), 0x5A, dtype=torch.uint8, device="cuda")
    plan.run(_dev(src), dst, _dev(s))
    torch.cuda.synchronize()
    got = dst.cpu().numpy()

    def region(name, nb):
        return got[doff[name]:doff[name] + nb]

    np.testing.assert_array_equal(region("w", 24 * 80 * 2).view(np.uint16), oq.dequant_rows(w, s, None, 24, 80).reshape(-1))
    np.testing.assert_array_equal(region("b", 48).view(np.uint16), oq.cast_f32_bf16(b32))
    np.testing.assert_array_equal(region("n", 666).view(np.uint16), oq.cast_f32_bf16(nrm))
    np.testing.assert_array_equal(region("bf", 200).view(np.float32), oq.bf16_bits_to_f32(bf))
    np.testing.assert_array_equal(region("raw", 1001), raw)
    assert not region("z", 77).any()
    assert (got[:2] == 0x5A).all() and (got[pos:] == 0x5A).all()


@pytest.mark.parametrize("line_off", [8, 16, 24, 32, 48, 56])
def test_regions_starting_inside_a_destination_line(line_off):
    """Destinations that start inside a 64-byte line, where the plan places a lead of elements
    before each region so the tiles' spans start on lines: every kind, regions of several tiles with
    ragged ends, padded int8 rows, byte canaries between the regions."""
    rng = np.random.default_rng(line_off)
    w = rng.integers(-127, 128, (70, 3072), dtype=np.int8)          # several int8 tiles
    wp = rng.integers(-127, 128, (13, 104), dtype=np.int8)          # padded rows: 96 of 104 used
    ws = rng.integers(-127, 128, (9, 40), dtype=np.int8)            # fp32 out
    s = np.exp(rng.normal(-6, 0.5, 70 + 13 + 9)).astype(np.float32)
    f = rng.normal(0, 1, 5000).astype(np.float32)                   # cast, ragged end
    bf = oq.cast_f32_bf16(rng.normal(0, 1, 3000).astype(np.float32))
    raw = rng.integers(0, 256, 9000, dtype=np.uint8)
    src, (o_w, o_wp, o_ws, o_f, o_bf, o_raw) = _pack([w, wp, ws, f, bf, raw], start=line_off, align=16)
    sizes = [("w", 70 * 3072 * 2), ("wp", 13 * 96 * 2), ("ws", 9 * 40 * 4), ("f", 5000 * 2), ("bf", 3000 * 4),
             ("raw", 9000), ("z", 7000)]
    doff, pos = {}, 0
    for name, nb in sizes:
        pos = (pos + 63) // 64 * 64 + line_off    # every region starts line_off bytes into a line
        doff[name] = pos
        pos += nb
    descs = make_descs([
        (KIND_I8_ROWSCALE_BF16, o_w, doff["w"], 70, 3072, 0, 0),
        (KIND_I8_ROWSCALE_BF16, o_wp, doff["wp"], 13, 96, 104, 70),
        (KIND_I8_ROWSCALE_F32, o_ws, doff["ws"], 9, 40, 0, 83),
        (KIND_F32_BF16, o_f, doff["f"], 1, 5000, 0, 0),
        (KIND_BF16_F32, o_bf, doff["bf"], 1, 3000, 0, 0),
        (KIND_COPY_BYTES, o_raw, doff["raw"], 1, 9000, 0, 0),
        (KIND_ZERO_BYTES, 0, doff["z"], 1, 7000, 0, 0),
    ])
    dst = torch.full((pos + 64,), 0x5A, dtype=torch.uint8, device="cuda")
    UnpackPlan(descs).run(_dev(src), dst, _dev(s))
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    written = np.zeros(got.size, bool)

    def region(name, nb):
        written[doff[name]:doff[name] + nb] = True
        return got[doff[name]:doff[name] + nb]

    np.testing.assert_array_equal(region("w", 70 * 3072 * 2).view(np.uint16),
                                  oq.dequant_rows(w, s[:70], None, 70, 3072).reshape(-1))
    np.testing.assert_array_equal(region("wp", 13 * 96 * 2).view(np.uint16),
                                  oq.dequant_rows(wp, s[70:83], None, 13, 96).reshape(-1))
    np.testing.assert_array_equal(region("ws", 9 * 40 * 4).view(np.uint32),
                                  oq.dequant_rows(ws, s[83:], None, 9, 40, out="float32").view(np.uint32).reshape(-1))
    np.testing.assert_array_equal(region("f", 10000).view(np.uint16), oq.cast_f32_bf16(f))
    np.testing.assert_array_equal(region("bf", 12000).view(np.float32), oq.bf16_bits_to_f32(bf))
    np.testing.assert_array_equal(region("raw", 9000), raw)
    assert not region("z", 7000).any()
    assert (got[~written] == 0x5A).all(), "wrote outside its regions"


def test_cast_golden_vectors_including_nan():
    z = _golden("bf16_cast.npz")
    f = z["f32_bits"].view(np.float32)
    src, (o,) = _pack([f], start=4)
    plan = UnpackPlan(make_descs([(KIND_F32_BF16, o, 0, 1, f.size, 0, 0)]))
    dst = torch.empty(f.size, dtype=torch.bfloat16, device="cuda")
    unpack_cast_f32_bf16(plan, _dev(src).view(torch.uint8), dst)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u16(dst), z["bf16_bits"])


def test_cast_exhaustive_all_fp32_patterns():
    """All 2^32 fp32 bit patterns through the cast kernel against the closed form."""
    chunk = 1 << 28
    plan = UnpackPlan(make_descs([(KIND_F32_BF16, 0, 0, 1, chunk, 0, 0)]))
    dst = torch.empty(chunk, dtype=torch.bfloat16, device="cuda")
    for start in range(0, 1 << 32, chunk):
        u = torch.arange(start, start + chunk, dtype=torch.int64, device="cuda")
        u32 = torch.where(u >= 2**31, u - 2**32, u).to(torch.int32)
        unpack_cast_f32_bf16(plan, u32.view(torch.float32), dst)
        want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        is_nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
        want = torch.where(is_nan, torch.full_like(want, 0xFFFF), want)
        got = dst.view(torch.int16).to(torch.int64) & 0xFFFF
        bad = (got != want).nonzero()
        assert bad.numel() == 0, f"first mismatch at pattern {start + int(bad[0]):#010x}"
        del u, u32, want, is_nan, got


def test_config2_full_dequant_bit_exact():
    regions = config2_regions()
    plan = UnpackPlan(config2_descs(regions, "dequant"))
    src, scales = config2_device_inputs(regions, "dequant", seed=1234)
    n = sum(g.numel for g in regions)
    assert plan.info["elements"] == n == 2_210_302_856
    assert plan.info["algo_bytes"] == 6_633_232_696
    dst = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    dequant_i8_rowscale_bf16(plan, src, scales, dst)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    for g in regions:
        q = src[g.elem_off:g.elem_off + g.numel].view(g.rows, g.cols)
        s = scales[g.scale_off:g.scale_off + g.rows]
        want = (q.to(torch.float32) * s.unsqueeze(1)).to(torch.bfloat16)
        got = dst[g.elem_off:g.elem_off + g.numel].view(g.rows, g.cols)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"tensor {g.index} {g.rows}x{g.cols}"
        # the device checker itself against the oracle on sampled rows
        rows = rng.choice(g.rows, size=min(3, g.rows), replace=False)
        for r in rows:
            ref = oq.dequant_rows(q[r:r + 1].cpu().numpy(), s[r:r + 1].cpu().numpy(), None, 1, g.cols)
            np.testing.assert_array_equal(_u16(got[r]), ref.reshape(-1))


def test_config2_full_cast_bit_exact():
    regions = config2_regions()
    plan = UnpackPlan(config2_descs(regions, "cast"))
    src, _ = config2_device_inputs(regions, "cast", seed=99)
    n = sum(g.numel for g in regions)
    assert plan.info["algo_bytes"] == 13_261_817_136
    dst = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    unpack_cast_f32_bf16(plan, src, dst)
    torch.cuda.synchronize()
    assert torch.equal(dst.view(torch.int16), src.to(torch.bfloat16).view(torch.int16))
    idx = np.random.default_rng(1).integers(0, n, 4096)
    np.testing.assert_array_equal(_u16(dst[idx]), oq.cast_f32_bf16(src[idx].cpu().numpy()))


def test_launch_on_side_stream_and_repeat():
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, (300, 3072), dtype=np.int8)
    s = np.exp(rng.normal(-6, 0.5, 300)).astype(np.float32)
    plan = UnpackPlan(make_descs([(KIND_I8_ROWSCALE_BF16, 0, 0, 300, 3072, 0, 0)]))
    src, sc = _dev(q), _dev(s)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    outs = []
    for _ in range(3):
        dst = torch.empty(300 * 3072, dtype=torch.bfloat16, device="cuda")
        with torch.cuda.stream(side):
            dequant_i8_rowscale_bf16(plan, src, sc, dst, stream=side)
        outs.append(dst)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = oq.dequant_rows(q, s, None, 300, 3072).reshape(-1)
    for d in outs:
        np.testing.assert_array_equal(_u16(d), want)


def test_entry_points_reject_bad_buffers_before_launch():
    plan = UnpackPlan(make_descs([(KIND_I8_ROWSCALE_BF16, 0, 0, 4, 16, 0, 0)]))
    src = torch.zeros(64, dtype=torch.int8, device="cuda")
    sc = torch.ones(4, device="cuda")
    with pytest.raises(ValueError, match="destination"):
        dequant_i8_rowscale_bf16(plan, src, sc, torch.empty(63, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="source"):
        dequant_i8_rowscale_bf16(plan, src[:63], sc, torch.empty(64, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="scales"):
        dequant_i8_rowscale_bf16(plan, src, sc[:3], torch.empty(64, dtype=torch.bfloat16, device="cuda"))
    cast_plan = UnpackPlan(make_descs([(KIND_F32_BF16, 0, 0, 1, 16, 0, 0)]))
    with pytest.raises(ValueError, match="kinds"):
        dequant_i8_rowscale_bf16(cast_plan, src, sc, torch.empty(64, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="kinds"):
        unpack_cast_f32_bf16(plan, src, torch.empty(64, dtype=torch.bfloat16, device="cuda"))
    empty = UnpackPlan(make_descs([]))
    empty.run(None, torch.empty(1, dtype=torch.uint8, device="cuda"))
