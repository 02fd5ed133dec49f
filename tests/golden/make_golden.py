"""Writes the golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Expected outputs come from torch's CPU kernels — the library whose arithmetic
the reference calls for this path (src/stagehand/scheduler.py:181, 299-300,
305, 1071) — on seeded inputs, plus the reference's own known-answer case
(tests/test_scheduler.py:307-373). The reference itself is not imported.
Fixtures are small .npz files: inputs and expected bit patterns only.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent
SEED = 20261201


def bf16_bits_torch(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def f32_from_bits(u) -> np.ndarray:
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def edge_f32_patterns() -> np.ndarray:
    pats: list[int] = []
    for sign in (0, 0x80000000):
        for exp in (0, 1, 2, 0x3F, 0x7F, 0x80, 0xFD, 0xFE, 0xFF):
            for mant in (0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x10000, 0x17FFF, 0x18000, 0x18001,
                         0x3FFFFF, 0x400000, 0x7F7FFF, 0x7F8000, 0x7FFFFF):
                pats.append(sign | (exp << 23) | mant)
    return np.array(sorted(set(pats)), dtype=np.uint32)


def main() -> None:
    rng = np.random.default_rng(SEED)

    # 1. fp32 → bf16: edge patterns + random patterns (all exponents) + N(0, 0.02).
    edges = edge_f32_patterns()
    rand_bits = rng.integers(0, 2**32, size=16384, dtype=np.uint64).astype(np.uint32)
    normal = rng.normal(0.0, 0.02, size=16384).astype(np.float32).view(np.uint32)
    bits = np.concatenate([edges, rand_bits, normal])
    np.savez_compressed(OUT / "bf16_cast.npz", f32_bits=bits, bf16_bits=bf16_bits_torch(f32_from_bits(bits)))

    # 2. The reference's SquareQ known-answer case (tests/test_scheduler.py:307-373):
    #    qweight = arange(64, int8).reshape(8, 8) - 32, scale = 1, zero_point = 0, bias = arange(8).
    q = (torch.arange(64, dtype=torch.int8).reshape(8, 8) - 32).contiguous()
    scale = torch.ones(8, dtype=torch.float32)
    zp = torch.zeros(8, dtype=torch.float32)
    bias = torch.arange(8, dtype=torch.float32)
    deq = (q.to(torch.float32) - zp.unsqueeze(1)) * scale.unsqueeze(1)
    np.savez_compressed(
        OUT / "squareq_known_answer.npz",
        qweight=q.numpy(), scale=scale.numpy(), zero_point=zp.numpy(), bias=bias.numpy(),
        weight_f32=deq.numpy(),
        weight_bf16_bits=deq.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16),
        bias_bf16_bits=bias.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16),
    )

    # 3. Row samples of the config-2 shapes: q ~ U{-127..127}, s = exp(N(-6, 0.5)) per row;
    #    plus an edge block with special scales and zero points.
    g = torch.Generator().manual_seed(SEED)
    arrays: dict[str, np.ndarray] = {}
    for i, (rows, cols) in enumerate([(4, 3072), (3, 12288), (5, 3072), (64, 1), (7, 77)]):
        qq = torch.randint(-127, 128, (rows, cols), dtype=torch.int8, generator=g)
        ss = torch.exp(torch.randn(rows, generator=g) * 0.5 - 6.0).to(torch.float32)
        zz = torch.zeros(rows, dtype=torch.float32)
        out = ((qq.to(torch.float32) - zz.unsqueeze(1)) * ss.unsqueeze(1)).to(torch.bfloat16)
        arrays[f"q{i}"] = qq.numpy()
        arrays[f"s{i}"] = ss.numpy()
        arrays[f"out{i}"] = out.view(torch.int16).numpy().view(np.uint16)
    special = np.array(
        [1.0, 2.0**-126, 2.0**-149, 1e-45, 3.0e-39, 2.0**-10, 0.5, 3.0e38, 3.4028235e38, -1.5,
         -2.0**-140, 0.0, -0.0, np.inf, -np.inf, np.nan, 7.3e-3, 1.0 / 3.0],
        dtype=np.float32)
    qall = np.arange(-128, 128, dtype=np.int8)
    qe = torch.from_numpy(np.tile(qall, (special.size, 1)))
    se = torch.from_numpy(special)
    ze = torch.from_numpy(np.array([0.0, 0.0, 0.0, 1.0, -3.0, 0.25, 0.0, 0.0, 0.0, 0.0,
                                    0.0, 5.0, 0.0, 0.0, 0.0, 0.0, 127.0, -0.5], dtype=np.float32))
    oe = ((qe.to(torch.float32) - ze.unsqueeze(1)) * se.unsqueeze(1)).to(torch.bfloat16)
    arrays["q_edge"] = qe.numpy()
    arrays["s_edge"] = special
    arrays["z_edge"] = ze.numpy()
    arrays["out_edge"] = oe.view(torch.int16).numpy().view(np.uint16)
    arrays["outf32_edge"] = ((qe.to(torch.float32) - ze.unsqueeze(1)) * se.unsqueeze(1)).numpy()
    np.savez_compressed(OUT / "squareq_rows.npz", **arrays)
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()
