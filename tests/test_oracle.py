"""Pins the CPU oracle (oracle/squareq.py) before it is trusted as the checker.

Each oracle function is checked against something it does not restate:
golden vectors written by torch's CPU kernels (tests/golden/make_golden.py),
the reference's own known-answer case (tests/test_scheduler.py:294-375),
exact rational arithmetic, and an exhaustive sweep of all 2^32 fp32 patterns
against torch's conversion. The mutant tests show that plausible mistakes
(truncation instead of rounding, a dropped tie term, a transposed scale
index, an FMA-style reassociation) fail these pins.
"""
from __future__ import annotations

import os
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import squareq as oq

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ── exact rounding, written independently of the bit trick ─────────────────

def _bf16_exact(x: float) -> int:
    """Nearest bf16 (8 significant bits, ties to even) of a finite fp32 value, by rational arithmetic."""
    if x == 0.0:
        return 0x8000 if np.signbit(x) else 0x0000
    sign = 0x8000 if x < 0 else 0
    v = Fraction(abs(x))
    # bf16: exponent bias 127, 7 stored mantissa bits, subnormal quantum 2^-133.
    e = v.numerator.bit_length() - v.denominator.bit_length()
    if Fraction(2) ** e > v:
        e -= 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 7)
    k, rem = divmod(v, quantum)
    k = int(k)
    if rem > quantum / 2 or (rem == quantum / 2 and k % 2 == 1):
        k += 1
    val = k * quantum
    max_finite = Fraction(2) ** 127 * Fraction(255, 128)
    if val > max_finite:
        return sign | 0x7F80
    # Encode val (exact bf16 value) as bits through fp32 (exact).
    f = np.float32(float(val))
    return sign | int((np.array([f], dtype=np.float32).view(np.uint32)[0] >> 16) & 0x7FFF)


def test_bf16_matches_golden_torch_vectors():
    z = _load("bf16_cast.npz")
    f = z["f32_bits"].view(np.float32)
    got = oq.bf16_rne_bits(f)
    np.testing.assert_array_equal(got, z["bf16_bits"])


def test_bf16_matches_exact_rational_rounding():
    z = _load("bf16_cast.npz")
    f = z["f32_bits"].view(np.float32)
    finite = f[np.isfinite(f)][:6000]
    got = oq.bf16_rne_bits(finite)
    want = np.array([_bf16_exact(float(x)) for x in finite], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)
    # infinities and NaN
    specials = np.array([np.inf, -np.inf, np.nan, -np.nan], dtype=np.float32)
    np.testing.assert_array_equal(oq.bf16_rne_bits(specials), np.array([0x7F80, 0xFF80, 0xFFFF, 0xFFFF], dtype=np.uint16))


@pytest.mark.slow
def _bf16_first_mismatch(start: int, count: int) -> int | None:
    u = np.arange(start, start + count, dtype=np.uint32)
    f = u.view(np.float32)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    bad = np.flatnonzero(oq.bf16_rne_bits(f) != want)
    return None if bad.size == 0 else int(u[bad[0]])


def test_bf16_exhaustive_against_torch():
    """All 2^32 fp32 bit patterns: the oracle equals torch's CPU conversion (chunks on threads:
    numpy and torch release the GIL in these loops)."""
    import concurrent.futures

    chunk = 1 << 22
    starts = range(0, 1 << 32, chunk)
    with concurrent.futures.ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        for start, bad in zip(starts, ex.map(_bf16_first_mismatch, starts, [chunk] * len(starts))):
            assert bad is None, f"chunk {start:#x}: first mismatch at {bad:#010x}"


# ── dequant ────────────────────────────────────────────────────────────────

def test_dequant_reference_known_answer():
    """tests/test_scheduler.py:307-373 of the reference: scale 1, zero point 0, q = arange(64)-32."""
    z = _load("squareq_known_answer.npz")
    w32 = oq.dequant_rows(z["qweight"], z["scale"], z["zero_point"], 8, 8, out="float32")
    np.testing.assert_array_equal(w32, z["qweight"].astype(np.float32))
    np.testing.assert_array_equal(w32, z["weight_f32"])
    wbf = oq.dequant_rows(z["qweight"], z["scale"], z["zero_point"], 8, 8, out="bfloat16")
    np.testing.assert_array_equal(wbf, z["weight_bf16_bits"])
    # |q| <= 32 is exact in bf16: the bf16 result widens back to q.
    np.testing.assert_array_equal(oq.bf16_bits_to_f32(wbf), z["qweight"].astype(np.float32))
    np.testing.assert_array_equal(oq.cast_f32_bf16(z["bias"]), z["bias_bf16_bits"])


def test_dequant_rows_match_golden():
    z = _load("squareq_rows.npz")
    for i in range(5):
        q, s = z[f"q{i}"], z[f"s{i}"]
        got = oq.dequant_rows(q, s, np.zeros_like(s), q.shape[0], q.shape[1])
        np.testing.assert_array_equal(got, z[f"out{i}"], err_msg=f"shape {q.shape}")
        # zero points absent == zero points of 0.0
        np.testing.assert_array_equal(oq.dequant_rows(q, s, None, q.shape[0], q.shape[1]), got)
    got = oq.dequant_rows(z["q_edge"], z["s_edge"], z["z_edge"], *z["q_edge"].shape)
    np.testing.assert_array_equal(got, z["out_edge"])
    got32 = oq.dequant_rows(z["q_edge"], z["s_edge"], z["z_edge"], *z["q_edge"].shape, out="float32")
    np.testing.assert_array_equal(got32.view(np.uint32), z["outf32_edge"].view(np.uint32))


def test_dequant_bruteforce_exact():
    """Every int8 value x a scale sweep: fp32 product (exact in double, rounded once) then exact bf16."""
    q = np.arange(-128, 128, dtype=np.int8)
    scales = np.concatenate([
        np.geomspace(1e-44, 3e38, 300).astype(np.float32),
        np.exp(np.random.default_rng(5).normal(-6.0, 0.5, 200)).astype(np.float32),
        np.array([1.0, 0.5, 2.0**-126, 2.0**-149, -1.0, -7.5e-3], dtype=np.float32),
    ])
    zps = np.zeros_like(scales)
    got = oq.dequant_rows(np.tile(q, (scales.size, 1)), scales, zps, scales.size, q.size)
    for r, s in enumerate(scales):
        for c, qq in enumerate(q):
            prod32 = np.float32(float(qq) * float(s))  # exact double product, one rounding to fp32
            want = 0xFFFF if np.isnan(prod32) else (
                (0x7F80 | (0x8000 if prod32 < 0 else 0)) if np.isinf(prod32) else _bf16_exact(float(prod32)))
            assert got[r, c] == want, (int(qq), float(s))


def test_dequant_matches_torch_expression_seeded():
    g = torch.Generator().manual_seed(7)
    q = torch.randint(-127, 128, (33, 100), dtype=torch.int8, generator=g)
    s = torch.exp(torch.randn(40, generator=g) * 0.5 - 6.0)
    zp = torch.randn(40, generator=g)
    want = ((q[:33, :96].to(torch.float32) - zp[:33].unsqueeze(1)) * s[:33].unsqueeze(1)).to(torch.bfloat16)
    got = oq.dequant_rows(q.numpy(), s.numpy(), zp.numpy(), 33, 96)
    np.testing.assert_array_equal(got, want.view(torch.int16).numpy().view(np.uint16))


# ── mutants: plausible mistakes must fail the pins ─────────────────────────

def _mutant_truncate(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _mutant_no_tie_even(x):
    u = np.asarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x8000)) >> 16).astype(np.uint16)


def test_pins_reject_rounding_mutants():
    z = _load("bf16_cast.npz")
    f = z["f32_bits"].view(np.float32)
    ok = ~np.isnan(f)
    for mutant in (_mutant_truncate, _mutant_no_tie_even):
        assert np.any(mutant(f)[ok] != z["bf16_bits"][ok]), mutant.__name__


def test_pins_reject_dequant_mutants():
    z = _load("squareq_rows.npz")
    q, s = z["q0"], z["s0"]
    want = z["out0"]
    # scale indexed by column instead of row
    bad1 = oq.bf16_rne_bits(q.astype(np.float32) * np.resize(s, q.shape[1])[None, :])
    assert np.any(bad1 != want)
    # edge block: q*s - z*s instead of (q - z)*s
    qe, se, ze = z["q_edge"], z["s_edge"], z["z_edge"]
    with np.errstate(all="ignore"):
        bad2 = oq.bf16_rne_bits(qe.astype(np.float32) * se[:, None] - (ze * se)[:, None])
    assert np.any(bad2 != z["out_edge"])


# ── layout and staging ─────────────────────────────────────────────────────

def test_layout_prefix_sums_config1():
    """8 x Linear(4096, 4096): W at 0 (33,554,432 B), bias at 33,554,432 (8,192 B) per layer."""
    lay = oq.build_param_layout([("weight", (4096, 4096)), ("bias", (4096,))], "bfloat16")
    assert [(e.name, e.offset, e.nbytes) for e in lay] == [("weight", 0, 33554432), ("bias", 33554432, 8192)]
    assert lay[-1].offset + lay[-1].nbytes == 33562624
    assert 8 * 33562624 == 268500992


def test_layout_no_padding_and_order():
    shapes = [("a", (3, 5)), ("b", (7,)), ("c", (1, 1)), ("d", (2, 3, 4))]
    lay = oq.build_param_layout(shapes, "bfloat16")
    off = 0
    for (name, shape), e in zip(shapes, lay):
        assert e.name == name and e.offset == off
        off += int(np.prod(shape)) * 2


def test_flatten_roundtrip():
    rng = np.random.default_rng(1)
    params = {"w": rng.normal(0, 0.02, (6, 10)).astype(np.float32), "b": rng.normal(0, 1, (6,)).astype(np.float32)}
    lay = oq.build_param_layout([("w", (6, 10)), ("b", (6,))], "bfloat16")
    buf = oq.flatten_params(params, lay)
    for e in lay:
        region = np.frombuffer(bytes(buf[e.offset:e.offset + e.nbytes]), dtype=np.uint16)
        np.testing.assert_array_equal(region, oq.cast_f32_bf16(params[e.name]))


def test_stage_squareq_block_branches():
    """Closed forms of each branch of _copy_squareq_backed_params_into_buffer (scheduler.py:243-325)."""
    rng = np.random.default_rng(3)
    out_f, in_f, padded = 6, 10, 16
    q = rng.integers(-127, 128, (out_f, padded), dtype=np.int8)
    s = np.exp(rng.normal(-6, 0.5, out_f)).astype(np.float32)
    zpt = rng.normal(0, 2, out_f).astype(np.float32)
    bias = rng.normal(0, 1, out_f).astype(np.float32)
    norm = rng.normal(1, 0.1, in_f).astype(np.float32)
    # nozp: the layer has qweight and scale but no zero_point, and the weight is a module
    # parameter: the module's value, cast (scheduler.py:272-275 fall through to 310), not a
    # dequant with a zero point of 0. notdict: the layer is not a dict: module parameter, then,
    # once evicted, the block's cache (scheduler.py:267, 310-322).
    live = rng.normal(0, 0.02, (out_f, in_f)).astype(np.float32)
    nd_live = rng.normal(0, 0.02, (4, 5)).astype(np.float32)
    nd_cached = rng.normal(0, 0.02, (4, 5)).astype(np.float32)
    shapes = [("lin.weight", (out_f, in_f)), ("lin.bias", (out_f,)), ("norm.weight", (in_f,)),
              ("gone.weight", (out_f, in_f)), ("nob.bias", (out_f,)), ("evicted.weight", (3,)),
              ("nozp.weight", (out_f, in_f)), ("nd.weight", (4, 5)), ("nd2.weight", (4, 5))]
    lay = oq.build_param_layout(shapes, "bfloat16")
    specs = {
        "lin.weight": oq.SquareQSpec("lin.weight", "lin", "weight", out_f, in_f, padded),
        "lin.bias": oq.SquareQSpec("lin.bias", "lin", "bias", out_f, in_f, padded),
        "gone.weight": oq.SquareQSpec("gone.weight", "missing_layer", "weight", out_f, in_f, padded),
        "nob.bias": oq.SquareQSpec("nob.bias", "nobias", "bias", out_f, in_f, padded),
        "nozp.weight": oq.SquareQSpec("nozp.weight", "nozp", "weight", out_f, in_f, padded),
        "nd.weight": oq.SquareQSpec("nd.weight", "notdict", "weight", 4, 5, 5),
        "nd2.weight": oq.SquareQSpec("nd2.weight", "notdict", "weight", 4, 5, 5),
    }
    layers = {"lin": {"qweight": q, "scale": s, "zero_point": zpt, "bias": bias}, "nobias": {},
              "nozp": {"qweight": q, "scale": s}, "notdict": np.ones(3, np.float32)}
    cache = {"evicted.weight": np.array([1.0, 2.0, 3.0], np.float32), "nd2.weight": nd_cached}
    buf = oq.stage_squareq_block(
        lay, specs, {"norm.weight", "evicted.weight", "nozp.weight", "nd.weight", "nd2.weight"},
        {"norm.weight": norm, "evicted.weight": np.zeros(0, np.float32), "nozp.weight": live, "nd.weight": nd_live,
         "nd2.weight": np.zeros(0, np.float32)}, layers, cache)
    region = {e.name: np.frombuffer(bytes(buf[e.offset:e.offset + e.nbytes]), np.uint16) for e in lay}
    # padded_in columns dropped, (q - zp) * s per row, rounded to bf16
    want_w = oq.bf16_rne_bits(((q[:, :in_f].astype(np.float32) - zpt[:, None]) * s[:, None]).astype(np.float32))
    np.testing.assert_array_equal(region["lin.weight"], want_w.reshape(-1))
    np.testing.assert_array_equal(region["lin.bias"], oq.cast_f32_bf16(bias))
    np.testing.assert_array_equal(region["norm.weight"], oq.cast_f32_bf16(norm))
    assert "norm.weight" in cache  # cached on first staging (scheduler.py:316-318)
    assert not region["gone.weight"].any()  # missing layer, not module-backed → zero fill
    assert not region["nob.bias"].any()  # bias spec without bias → zero fill
    np.testing.assert_array_equal(region["evicted.weight"], oq.cast_f32_bf16(cache["evicted.weight"]))
    # the module branch casts with torch's conversion, the library the reference calls
    torch_bf16 = lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    np.testing.assert_array_equal(region["nozp.weight"], torch_bf16(live).reshape(-1))
    dequant_zero_zp = oq.bf16_rne_bits((q[:, :in_f].astype(np.float32) * s[:, None]).astype(np.float32))
    assert not np.array_equal(region["nozp.weight"], dequant_zero_zp.reshape(-1))  # not a dequant with zp = 0
    np.testing.assert_array_equal(region["nd.weight"], torch_bf16(nd_live).reshape(-1))
    np.testing.assert_array_equal(region["nd2.weight"], torch_bf16(nd_cached).reshape(-1))
    assert "nd.weight" in cache and "nozp.weight" in cache


# ── oracle/torch_ref.py: the timed CPU baseline computes the checked values ─────

def test_torch_ref_host_dequant_matches_golden_rows():
    """``host_dequant_into`` (the reference's torch op sequence, scheduler.py:290-300, which the
    bench times as the CPU baseline) writes the golden rows' bf16 patterns, at unaligned slab
    offsets and with padded source rows."""
    from oracle import torch_ref

    z = _load("squareq_rows.npz")
    cases = [(z[f"q{i}"], z[f"s{i}"], np.zeros_like(z[f"s{i}"]), z[f"out{i}"]) for i in range(5)]
    cases.append((z["q_edge"], z["s_edge"], z["z_edge"], z["out_edge"]))
    regions, off, want = [], 3, []
    for q, s, zp, out in cases:
        rows, cols = out.shape
        padded = np.concatenate([q, np.full((rows, 5), 99, np.int8)], axis=1)  # padded_in columns are dropped
        regions.append((off, torch.from_numpy(padded), torch.from_numpy(s), torch.from_numpy(zp), rows, cols))
        want.append((off, out))
        off += 2 * out.size + 6
    slab = torch.full((off,), 0xA5, dtype=torch.uint8)
    torch_ref.host_dequant_into(slab, regions)
    raw = slab.numpy()
    for o, out in want:
        got = raw[o:o + 2 * out.size].view(np.uint16).reshape(out.shape)
        assert np.array_equal(got, out)
    assert (raw[:3] == 0xA5).all()  # nothing written outside the regions


def test_torch_ref_host_cast_matches_golden_patterns():
    """``host_cast_into`` (scheduler.py:181 / 1071) writes the golden bf16 patterns of every
    non-NaN fp32 input, and agrees with ``cast_f32_bf16`` on a seeded config-2-like tensor."""
    from oracle import torch_ref

    z = _load("bf16_cast.npz")
    f = z["f32_bits"].view(np.float32)
    keep = ~np.isnan(f)
    src = f[keep]
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((77, 1000)) * 0.02).astype(np.float32)
    slab = torch.zeros(2 * (src.size + w.size) + 2, dtype=torch.uint8)
    torch_ref.host_cast_into(slab, [(0, torch.from_numpy(src)), (2 * src.size + 2, torch.from_numpy(w))])
    raw = slab.numpy()
    assert np.array_equal(raw[:2 * src.size].view(np.uint16), z["bf16_bits"][keep])
    assert np.array_equal(raw[2 * src.size + 2:].view(np.uint16), oq.cast_f32_bf16(w))
