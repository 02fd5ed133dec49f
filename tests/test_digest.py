"""Chunk digests (``sh_block_digest`` / ``sh_block_changed`` / ``sh_block_digest_host``), the basis
of save-backs that copy back only the chunks a block changed on the device.

The digest has no counterpart in the reference (which copies every block back whole,
src/stagehand/scheduler.py:1216-1226); what has to hold is that a changed chunk is seen. The CPU
tests pin the host function to the definition in ``sh_digest.cpp`` (restated with numpy below),
and check that changing any one byte changes exactly the digest of the chunk holding it. The GPU
tests check that the device kernels compute the host function's digests and flags.
"""
from __future__ import annotations

import numpy as np
import pytest

from stagehand_amd import _native

M64 = (1 << 64) - 1
KEY = 0x9E3779B9


def _mix32(x: np.ndarray, s1: int, m1: int, s2: int, m2: int, s3: int) -> np.ndarray:
    x = (x ^ (x >> np.uint32(s1))) * np.uint32(m1)
    x = (x ^ (x >> np.uint32(s2))) * np.uint32(m2)
    return x ^ (x >> np.uint32(s3))


def digest_np(buf: np.ndarray, chunk: int) -> np.ndarray:
    """The digest as sh_digest.cpp defines it: per chunk, the sums mod 2^64 over its 8-byte words
    w_j (j = byte offset / 8, the last word zero-padded; l, h its 32-bit halves, k = j*KEY mod
    2^32) of f(l^k) + f(h^k)*2^32 and g(l^k) + g(h^k)*2^32, with f MurmurHash3's fmix32 and g
    lowbias32."""
    n = buf.size
    padded = np.zeros(-(-n // 8) * 8, np.uint8)
    padded[:n] = buf
    halves = padded.view("<u4").astype(np.uint32).reshape(-1, 2)
    j = np.arange(halves.shape[0], dtype=np.uint64)
    k = ((j * np.uint64(KEY)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    lo, hi = halves[:, 0] ^ k, halves[:, 1] ^ k
    with np.errstate(over="ignore"):
        f = [_mix32(v, 16, 0x85EBCA6B, 13, 0xC2B2AE35, 16).astype(np.uint64) for v in (lo, hi)]
        g = [_mix32(v, 16, 0x7FEB352D, 15, 0x846CA68B, 16).astype(np.uint64) for v in (lo, hi)]
    a = f[0] | (f[1] << np.uint64(32))
    b = g[0] | (g[1] << np.uint64(32))
    n_chunks = -(-n // chunk)
    out = np.zeros(2 * n_chunks, np.uint64)
    per = chunk // 8
    for c in range(n_chunks):
        out[2 * c] = int(a[c * per:(c + 1) * per].astype(object).sum()) & M64
        out[2 * c + 1] = int(b[c * per:(c + 1) * per].astype(object).sum()) & M64
    return out


def test_mixers_match_their_published_values():
    """fmix32 and lowbias32 at known points: fmix32(0) = 0, and both are the published functions
    (values computed from their definitions in exact integer arithmetic)."""
    def ref(x, s1, m1, s2, m2, s3):
        x ^= x >> s1
        x = (x * m1) & 0xFFFFFFFF
        x ^= x >> s2
        x = (x * m2) & 0xFFFFFFFF
        return x ^ (x >> s3)

    xs = np.array([0, 1, 2, 0xFFFFFFFF, 0x12345678, 0x80000000], np.uint32)
    with np.errstate(over="ignore"):
        got_f = _mix32(xs, 16, 0x85EBCA6B, 13, 0xC2B2AE35, 16)
        got_g = _mix32(xs, 16, 0x7FEB352D, 15, 0x846CA68B, 16)
    assert [int(v) for v in got_f] == [ref(int(x), 16, 0x85EBCA6B, 13, 0xC2B2AE35, 16) for x in xs]
    assert [int(v) for v in got_g] == [ref(int(x), 16, 0x7FEB352D, 15, 0x846CA68B, 16) for x in xs]
    assert int(got_f[0]) == 0 and int(got_f[1]) == 0x514E28B7  # MurmurHash3 fmix32(1)


def test_mixers_are_bijections_on_a_sample():
    """Invertibility on a sample of 2^20 inputs: no two map to the same output."""
    xs = np.arange(1 << 20, dtype=np.uint32) * np.uint32(0x9E3779B1)
    with np.errstate(over="ignore"):
        for params in ((16, 0x85EBCA6B, 13, 0xC2B2AE35, 16), (16, 0x7FEB352D, 15, 0x846CA68B, 16)):
            assert np.unique(_mix32(xs, *params)).size == xs.size


def digest_host(buf: np.ndarray, chunk: int) -> np.ndarray:
    out = np.zeros(2 * max(1, -(-buf.size // chunk)), np.uint64)
    assert _native.lib().sh_block_digest_host(buf.ctypes.data if buf.size else None, buf.size, chunk,
                                              out.ctypes.data) == _native.SH_OK, _native.last_error()
    return out[:2 * -(-buf.size // chunk)]


@pytest.mark.parametrize("n,chunk", [(1, 16), (15, 16), (16, 16), (17, 16), (100, 32), (4096, 4096),
                                     (4104, 4096), (3 * 4096 + 5, 4096), (65536 + 9, 1024)])
def test_host_digest_is_the_stated_function(n, chunk):
    rng = np.random.default_rng(n * 31 + chunk)
    buf = rng.integers(0, 256, n, dtype=np.uint8)
    np.testing.assert_array_equal(digest_host(buf, chunk), digest_np(buf, chunk))


def test_zero_bytes_make_no_chunks():
    out = np.full(2, 7, np.uint64)
    assert _native.lib().sh_block_digest_host(None, 0, 4096, out.ctypes.data) == _native.SH_OK
    assert (out == 7).all()


def test_every_single_byte_change_changes_only_its_chunk():
    """Each step of the digest is a bijection of a 64-bit word, so changing one word always changes
    its chunk's digest (no probability involved), and leaves every other chunk's alone."""
    rng = np.random.default_rng(5)
    chunk = 256
    buf = rng.integers(0, 256, 10 * chunk + 37, dtype=np.uint8)
    base = digest_host(buf, chunk)
    positions = list(rng.integers(0, buf.size, 300)) + [0, chunk - 1, chunk, buf.size - 1, 10 * chunk]
    for pos in positions:
        for delta in (1, 128, 255):
            mod = buf.copy()
            mod[pos] ^= delta
            d = digest_host(mod, chunk)
            c = pos // chunk
            assert (d[2 * c] != base[2 * c]) and (d[2 * c + 1] != base[2 * c + 1]), (pos, delta)
            others = np.ones(d.size, bool)
            others[2 * c:2 * c + 2] = False
            np.testing.assert_array_equal(d[others], base[others])


def test_swapped_and_cancelling_changes_are_seen():
    """Changes that a plain sum or xor of the words would miss: two words swapped, one word
    raised and another lowered by the same amount, a word moved within its chunk."""
    rng = np.random.default_rng(6)
    chunk = 4096
    buf = rng.integers(0, 256, 4 * chunk, dtype=np.uint8)
    base = digest_host(buf, chunk)
    w = buf.view("<u8")
    swapped = w.copy()
    swapped[[3, 9]] = swapped[[9, 3]]
    cancel = w.copy()
    cancel[5] += np.uint64(1000)
    cancel[6] -= np.uint64(1000)
    moved = w.copy()
    moved[20:40] = np.roll(moved[20:40], 1)
    for mod in (swapped, cancel, moved):
        d = digest_host(mod.view(np.uint8), chunk)
        assert d[0] != base[0] and d[1] != base[1]
        np.testing.assert_array_equal(d[2:], base[2:])


def test_arguments_are_checked():
    lib = _native.lib()
    buf = np.zeros(64, np.uint8)
    out = np.zeros(16, np.uint64)
    assert lib.sh_block_digest_host(buf.ctypes.data, 64, 0, out.ctypes.data) == _native.SH_ERR_INVALID
    assert lib.sh_block_digest_host(buf.ctypes.data, 64, 24, out.ctypes.data) == _native.SH_ERR_INVALID
    assert b"multiple of 16" in lib.sh_last_error()
    assert lib.sh_block_digest_host(None, 64, 16, out.ctypes.data) == _native.SH_ERR_INVALID
    assert lib.sh_block_digest_host(buf.ctypes.data, 1 << 40, 16, out.ctypes.data) == _native.SH_ERR_INVALID


@pytest.mark.gpu
@pytest.mark.parametrize("n,chunk", [(17, 16), (4096 * 7 + 3, 4096), ((8 << 20) + 11, 1 << 20), (48 << 20, 1 << 20),
                                     ((1 << 20) - 16, 1 << 20)])
def test_device_digest_and_flags_match_the_host(n, chunk):
    import torch

    g = torch.Generator(device="cuda").manual_seed(n)
    dev = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    n_chunks = -(-n // chunk)
    dig = torch.zeros(2 * n_chunks, dtype=torch.int64, device="cuda")
    lib = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.sh_block_digest(dev.data_ptr(), n, chunk, dig.data_ptr(), stream) == _native.SH_OK
    torch.cuda.synchronize()
    want = digest_host(dev.cpu().numpy(), chunk)
    np.testing.assert_array_equal(dig.cpu().numpy().view(np.uint64), want)
    # unchanged: no flags; then change bytes in a few chunks, the last one included
    flags = torch.full((n_chunks + 8,), 7, dtype=torch.uint8, pin_memory=True)
    assert lib.sh_block_changed(dev.data_ptr(), n, chunk, dig.data_ptr(), flags.data_ptr(), stream) == _native.SH_OK
    torch.cuda.synchronize()
    assert not flags[:n_chunks].any() and (flags[n_chunks:] == 7).all()
    hit = sorted({0, n_chunks - 1, n_chunks // 2})
    for c in hit:
        pos = min(c * chunk + 5, n - 1)
        dev[pos] ^= 0x40
    assert lib.sh_block_changed(dev.data_ptr(), n, chunk, dig.data_ptr(), flags.data_ptr(), stream) == _native.SH_OK
    torch.cuda.synchronize()
    expect = np.zeros(n_chunks, np.uint8)
    expect[hit] = 1
    np.testing.assert_array_equal(flags[:n_chunks].numpy(), expect)


@pytest.mark.gpu
@pytest.mark.parametrize("offset", [1, 4, 8, 12])
def test_device_digest_of_a_buffer_at_any_byte_offset(offset):
    """The kernel reads 16-byte words at any alignment of the buffer's start."""
    import torch

    n, chunk = (3 << 20) + 21, 1 << 18
    g = torch.Generator(device="cuda").manual_seed(offset)
    base = torch.randint(0, 256, (n + 64,), dtype=torch.uint8, device="cuda", generator=g)
    dev = base[offset:offset + n]
    n_chunks = -(-n // chunk)
    dig = torch.zeros(2 * n_chunks, dtype=torch.int64, device="cuda")
    lib = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.sh_block_digest(dev.data_ptr(), n, chunk, dig.data_ptr(), stream) == _native.SH_OK
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dig.cpu().numpy().view(np.uint64), digest_host(dev.cpu().numpy(), chunk))
