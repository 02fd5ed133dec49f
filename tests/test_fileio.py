"""Native weight-file reader (sh_file_* and file ranges in block loads).

CPU cases check the reader itself against the file's bytes (buffered and
O_DIRECT reads, ranges across 8 MiB pieces, unaligned and empty ranges, error
statuses) and the slab layout SourceBuilder gives file ranges (file order,
merged neighbours), with the descriptor table applied on the CPU. GPU cases stream file-backed models with every
reader against the same model run unstreamed, bit for bit — the reference's
mmap reads (src/stagehand/scheduler.py:184-241, 564-601) are the "mmap" case.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle.squareq import cast_f32_bf16, dequant_rows
from stagehand_amd import _native
from stagehand_amd.fileio import ALIGN, FileCache, FileRange, WeightFile
from stagehand_amd.staging import SourceBuilder
from stagehand_amd.unpack import (KIND_BF16_F32, KIND_COPY_BYTES, KIND_F32_BF16, KIND_I8_ROWSCALE_BF16,
                                  KIND_ZERO_BYTES)


def _aligned(nbytes: int, misalign: int = 0) -> tuple[np.ndarray, torch.Tensor]:
    """A host byte tensor whose data pointer is ``misalign`` past a 4 KiB boundary."""
    raw = np.zeros(nbytes + 2 * ALIGN, dtype=np.uint8)
    start = (-raw.ctypes.data) % ALIGN + misalign
    view = raw[start:start + nbytes]
    return raw, torch.from_numpy(view)


@pytest.fixture()
def blob(tmp_path):
    rng = np.random.default_rng(7)
    data = rng.integers(0, 256, size=(19 << 20) + 1237, dtype=np.uint8)
    path = tmp_path / "blob.bin"
    data.tofile(path)
    return path, data


@pytest.mark.parametrize("direct", [False, True])
@pytest.mark.parametrize("misalign", [0, 8, 4095])
def test_read_whole_file(blob, direct, misalign):
    path, data = blob
    f = WeightFile(path, direct=direct)
    assert f.size == data.size
    _keep, dst = _aligned(data.size, misalign)
    f.read_into(dst, 0)
    assert np.array_equal(dst.numpy(), data)
    info = f.info()
    assert info["bytes_direct"] + info["bytes_bounced"] + info["bytes_buffered"] == data.size
    if direct and info["direct"]:
        if misalign == 0:
            # congruent destination in ordinary memory: the storage DMA writes everything
            # between 4 KiB file offsets, and only the unaligned tail goes through the page cache
            assert info["bytes_direct"] >= data.size - 2 * ALIGN and info["bytes_bounced"] == 0
        else:
            # no congruence: every byte goes around the page cache through the bounce buffer
            assert info["bytes_bounced"] == data.size and info["bytes_direct"] == 0
    if not direct:
        assert info["bytes_direct"] == info["bytes_bounced"] == 0
    f.close()


def test_cached_pages_are_read_without_blocking(blob):
    """A second buffered read of a file the page cache holds is served entirely by the
    non-blocking reads (no cold-read slot is taken)."""
    path, data = blob
    f = WeightFile(path)
    _keep, dst = _aligned(data.size)
    f.read_into(dst, 0)
    first = f.info()
    f.read_into(dst, 0)
    second = f.info()
    assert np.array_equal(dst.numpy(), data)
    assert second["bytes_buffered"] - first["bytes_buffered"] == data.size
    assert second["bytes_cached"] - first["bytes_cached"] == data.size
    f.close()


def test_cold_reads_in_sequential_runs(blob):
    """After the file's pages are dropped, the reads that miss the page cache go through the
    sequential cold-read runs (several descriptors) and still land every byte in place."""
    path, data = blob
    fd = os.open(path, os.O_RDONLY)
    os.fsync(fd)
    os.close(fd)
    f = WeightFile(path)
    f.advise_dontneed()
    rng = np.random.default_rng(5)
    spans = [(int(o), int(n)) for o, n in zip(rng.integers(0, data.size // 2, 6), rng.integers(1, data.size // 2, 6))]
    spans.append((0, data.size))
    total = sum(n for _o, n in spans)
    _keep, dst = _aligned(total)
    ranges = np.zeros(len(spans), dtype=_native.FILE_RANGE_DTYPE)
    cursor = 0
    for i, (off, n) in enumerate(spans):
        ranges[i] = (f.handle, off, n, cursor)
        cursor += n
    _native.call("sh_file_read_batch", ranges.ctypes.data, len(spans), dst.data_ptr(), 16)
    out, cursor = dst.numpy(), 0
    for off, n in spans:
        assert np.array_equal(out[cursor:cursor + n], data[off:off + n])
        cursor += n
    info = f.info()
    assert info["bytes_buffered"] == total
    assert info["bytes_cached"] < total  # the dropped pages came from storage
    f.close()


@pytest.mark.parametrize("direct", [False, True])
def test_read_ranges(blob, direct):
    """Ranges at random offsets and lengths, across 8 MiB pieces, empty ones included."""
    path, data = blob
    f = WeightFile(path, direct=direct)
    rng = np.random.default_rng(11)
    spans = [(0, 0), (data.size - 1, 1), ((8 << 20) - 5, 10), (ALIGN, 3 * ALIGN), (123, (9 << 20) + 77)]
    for _ in range(12):
        off = int(rng.integers(0, data.size))
        spans.append((off, int(rng.integers(0, data.size - off + 1))))
    total = sum(n for _o, n in spans)
    _keep, dst = _aligned(total + ALIGN * len(spans))
    ranges = np.zeros(len(spans), dtype=_native.FILE_RANGE_DTYPE)
    cursor, want = 0, []
    for i, (off, n) in enumerate(spans):
        cursor += (off - cursor) % ALIGN  # congruent placement: the direct reader can take the middles
        ranges[i] = (f.handle, off, n, cursor)
        want.append((cursor, data[off:off + n]))
        cursor += n
    _native.call("sh_file_read_batch", ranges.ctypes.data, len(spans), dst.data_ptr(), 8)
    out = dst.numpy()
    for pos, ref in want:
        assert np.array_equal(out[pos:pos + ref.size], ref)
    f.close()


def test_errors(blob, tmp_path):
    path, data = blob
    f = WeightFile(path)
    _keep, dst = _aligned(64)
    with pytest.raises(ValueError, match="past the end"):
        f.read_into(dst, data.size - 10, 64)
    with pytest.raises(ValueError):
        f.read_into(dst, 0, 65)  # larger than the destination
    with pytest.raises(ValueError):
        _native.call("sh_file_advise", f.handle, 0, 0, 99)
    f.advise_willneed(0, 1 << 20)
    f.advise_dontneed()
    f.read_into(dst, 5)
    assert np.array_equal(dst.numpy(), data[5:69])
    f.close()
    with pytest.raises(RuntimeError):
        f.read_into(dst, 0)
    with pytest.raises(OSError):
        WeightFile(tmp_path / "missing.bin")
    with pytest.raises(ValueError):
        WeightFile(tmp_path)  # a directory
    cache = FileCache()
    assert cache.get(str(path), False) is cache.get(str(path), False)
    assert cache.get(str(path), True) is not cache.get(str(path), False)
    cache.close()


def _apply_descs(slab: np.ndarray, descs: np.ndarray, dst_bytes: int, scale_off: int = -1,
                 zp_off: int = -1) -> np.ndarray:
    """CPU application of a descriptor table (the unpack kernel's contract); the int8 rows use
    the oracle's dequant with the per-row scales / zero points the table points at."""
    out = np.zeros(dst_bytes, dtype=np.uint8)
    for d in descs:
        kind, s, o, n = int(d["kind"]), int(d["src_off"]), int(d["dst_off"]), int(d["rows"]) * int(d["cols"])
        if kind == KIND_I8_ROWSCALE_BF16:
            rows, cols, ld, r0 = int(d["rows"]), int(d["cols"]), int(d["src_ld"]), int(d["scale_off"])
            q = slab[s:s + rows * ld].view(np.int8).reshape(rows, ld)
            sc = slab[scale_off + 4 * r0:scale_off + 4 * (r0 + rows)].copy().view(np.float32)
            zp = None if zp_off < 0 else slab[zp_off + 4 * r0:zp_off + 4 * (r0 + rows)].copy().view(np.float32)
            out[o:o + 2 * n] = dequant_rows(q, sc, zp, rows, cols).astype("<u2").reshape(-1).view(np.uint8)
        elif kind == KIND_COPY_BYTES:
            out[o:o + n] = slab[s:s + n]
        elif kind == KIND_ZERO_BYTES:
            out[o:o + n] = 0
        elif kind == KIND_F32_BF16:
            bits = cast_f32_bf16(slab[s:s + 4 * n].copy().view(np.float32))
            out[o:o + 2 * n] = bits.astype("<u2").view(np.uint8)
        elif kind == KIND_BF16_F32:
            b16 = slab[s:s + 2 * n].copy().view("<u2").astype(np.uint32) << 16
            out[o:o + 4 * n] = b16.astype("<u4").view(np.uint8)
        else:
            raise AssertionError(kind)
    return out


@pytest.mark.parametrize("direct", [False, True])
def test_builder_file_layout(tmp_path, direct):
    """File ranges land in file order, neighbours merge into one read, and the descriptor
    table maps the slab to the reference layout (torch's cast of each tensor)."""
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(3)
    tensors = {
        "b.w1": torch.randn(300, 129, generator=g).to(torch.bfloat16),
        "b.bias": torch.randn(77, generator=g).to(torch.bfloat16),
        "b.w2": torch.randn(64, 1000, generator=g),  # fp32: cast on the device
        "b.norm": torch.randn(3, generator=g).to(torch.bfloat16),
    }
    path = tmp_path / "b.safetensors"
    save_file(tensors, str(path))
    raw = path.read_bytes()
    hlen = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + hlen])
    base = 8 + hlen
    f = WeightFile(path, direct=direct)
    layout = [("b.w2", torch.float32), ("b.norm", torch.bfloat16), ("gap", None), ("b.w1", torch.bfloat16),
              ("b.bias", torch.bfloat16)]
    b = SourceBuilder(torch.bfloat16, 0)
    dst_off, want = 0, bytearray()
    for name, dt in layout:
        if dt is None:
            b.add_zero(dst_off, 50)
            want += bytes(50)
            dst_off += 50
            continue
        lo, hi = header[name]["data_offsets"]
        numel = tensors[name].numel()
        assert b.add_file_param(dst_off, FileRange(f, base + lo, hi - lo), dt, numel)
        want += tensors[name].to(torch.bfloat16).view(torch.uint8).numpy().tobytes()
        dst_off += numel * 2
    b.dst_bytes = dst_off
    src, descs = b.finish()
    assert descs is not None  # an fp32 tensor needs the cast kernel
    ranges = [(off, p) for off, p in src.pieces if isinstance(p, FileRange)]
    # the four tensors are adjacent in the file (w2 first: safetensors puts wider dtypes first)
    # and sorted into file order, so they merge into one range
    assert len(ranges) == 1 and ranges[0][1].nbytes == sum(h["data_offsets"][1] - h["data_offsets"][0]
                                                           for k, h in header.items() if k != "__metadata__")
    _keep, slab = _aligned(src.src_bytes)
    r = np.zeros(1, dtype=_native.FILE_RANGE_DTYPE)
    r[0] = (f.handle, ranges[0][1].offset, ranges[0][1].nbytes, ranges[0][0])
    _native.call("sh_file_read_batch", r.ctypes.data, 1, slab.data_ptr(), 4)
    out = _apply_descs(slab.numpy(), descs, dst_off)
    assert out.tobytes() == bytes(want)
    f.close()


def _slab_bytes(src) -> np.ndarray:
    """The source slab a loader would assemble: host pieces copied, file ranges read."""
    _keep, slab = _aligned(src.src_bytes)
    out = slab.numpy()
    for off, p in src.pieces:
        if isinstance(p, FileRange):
            p.file.read_into(torch.from_numpy(out[off:off + p.nbytes]), p.offset, p.nbytes)
        else:
            out[off:off + p.numel() * p.element_size()] = p.reshape(-1).view(torch.uint8).numpy()
    return out.copy()


@pytest.mark.parametrize("direct", [False, True])
def test_builder_squareq_v2_file_regions(tmp_path, direct):
    """SquareQ V2 layers as file ranges (int8 rows, scales, zero points) give the bytes of the same
    layers as host tensors, and those of the oracle's dequant of src/stagehand/scheduler.py:285-300."""
    from stagehand_amd.squareq_v2 import read_v2_layers, read_v2_locations, write_v2_slab

    g = torch.Generator().manual_seed(9)
    spec = {"a": (40, 33, 40, True), "b": (17, 64, 64, False), "c": (9, 5, 8, None)}  # out, in, ld, zp
    layers = {}
    for name, (out_f, in_f, ld, zp) in spec.items():
        t = {"qweight": torch.randint(-127, 128, (out_f, ld), dtype=torch.int8, generator=g),
             "scale": torch.exp(torch.randn(out_f, generator=g) * 0.5 - 6.0), "in_features": in_f,
             "bias": torch.randn(out_f, generator=g).to(torch.bfloat16)}
        if zp is not None:
            t["zero_point"] = torch.randn(out_f, generator=g) if zp else torch.zeros(out_f)
        layers[name] = t
    path = str(tmp_path / "slab.safetensors")
    manifest = write_v2_slab(path, layers)
    views = read_v2_layers(path, manifest, memoryview(open(path, "rb").read()))
    locs = read_v2_locations(path, manifest)
    f = WeightFile(path, direct=direct)
    module_norm = torch.randn(24, generator=g)  # fp32 module parameter between the layers
    builders = [SourceBuilder(torch.bfloat16, 0), SourceBuilder(torch.bfloat16, 0)]
    want = bytearray()
    for bi, b in enumerate(builders):
        dst = 0
        for name, (out_f, in_f, ld, zp) in spec.items():
            if bi == 0:
                L = views[name]
                b.add_dequant(dst, L["qweight"], in_f, L["scale"], L["zero_point"])
            else:
                q, s_, z = locs[name]["qweight"], locs[name]["scale"], locs[name].get("zero_point")
                zr = FileRange(f, z[0], z[1]) if (z is not None and zp) else None
                b.add_dequant_file(dst, FileRange(f, q[0], q[1]), out_f, ld, in_f, FileRange(f, s_[0], s_[1]), zr)
            dst += out_f * in_f * 2
            if bi == 0:
                b.add_param(dst, views[name]["bias"])
            else:
                bl = locs[name]["bias"]
                assert b.add_file_param(dst, FileRange(f, bl[0], bl[1]), bl[2], out_f)
            dst += out_f * 2
            b.add_param(dst, module_norm, mutable=True)
            dst += 24 * 2
            if bi == 0:
                L = layers[name]
                want += dequant_rows(L["qweight"].numpy(), L["scale"].numpy(),
                                     L["zero_point"].numpy() if "zero_point" in L else None,
                                     out_f, in_f).astype("<u2").tobytes()
                want += L["bias"].view(torch.uint8).numpy().tobytes()
                want += cast_f32_bf16(module_norm.numpy()).astype("<u2").tobytes()
        b.dst_bytes = dst
    outs = []
    for b in builders:
        src, descs = b.finish()
        outs.append(_apply_descs(_slab_bytes(src), descs, b.dst_bytes, src.scale_off, src.zp_off).tobytes())
    assert outs[0] == bytes(want)
    assert outs[1] == bytes(want)
    f.close()


def test_builder_direct_copy_layout_without_direct_io(tmp_path):
    """bf16 → bf16 from a buffered file keeps the kernel-free layout: ranges at their layout offsets."""
    data = (torch.arange(4096, dtype=torch.int16)).view(torch.bfloat16)
    path = tmp_path / "x.bin"
    data.view(torch.uint8).numpy().tofile(path)
    f = WeightFile(path)
    b = SourceBuilder(torch.bfloat16, 8192 + 16)
    assert b.add_file_param(16, FileRange(f, 0, 8192), torch.bfloat16, 4096)
    b.add_zero(0, 16)
    src, descs = b.finish()
    assert descs is None and src.src_bytes == 8192 + 16
    assert [(o, type(p).__name__) for o, p in src.pieces] == [(16, "FileRange"), (0, "Tensor")]
    assert not b.add_file_param(0, FileRange(f, 0, 4), torch.float16, 2)  # no raw-byte conversion from fp16
    f.close()


# ── GPU: streaming parity per reader ──────────────────────────────────────

def _config(**kw):
    from stagehand_amd.config import StagehandConfig

    base = dict(pinned_pool_mb=64, pinned_slab_mb=4, vram_high_watermark_mb=200000, vram_low_watermark_mb=100000,
                prefetch_window_blocks=2, telemetry_enabled=True, nan_inf_check=False, strict_bf16=False)
    base.update(kw)
    cfg = StagehandConfig(**base)
    cfg.telemetry_file = None
    return cfg


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view(torch.int16).cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("reader", ["pread", "direct"])
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_file_backed_streaming_per_reader(tmp_path, reader, src_dtype):
    import stagehand_amd as stagehand
    from tests.streaming_models import TinyStack, init_, save_safetensors

    model = init_(TinyStack(n=6, hidden=256, mlp=4))
    path = tmp_path / "tiny.safetensors"
    save_safetensors(model, path, src_dtype)
    ref = init_(TinyStack(n=6, hidden=256, mlp=4)).to(device="cuda", dtype=torch.bfloat16)
    model.requires_grad_(False)
    model = model.to(torch.bfloat16)
    base_mb = torch.cuda.memory_allocated() / 2**20
    # watermarks below one block: every block is evicted and read from the file again each step
    cfg = _config(file_reader=reader, vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb),
                  prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_file_backed(str(path)) == 6 * 4
    x = torch.randn(5, 256).to(torch.bfloat16).cuda()
    outs = []
    for step in range(3):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            outs.append(model(x))
        rt.end_step()
    with torch.no_grad():
        want = ref(x)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    files = rt.scheduler._weight_files.files()
    assert len(files) == 1
    info = files[0].info()
    # every step reads every block again (watermarks below one block)
    read = info["bytes_direct"] + info["bytes_bounced"] + info["bytes_buffered"]
    assert read >= 3 * 6 * 2 * 256 * 1024 * src_dtype.itemsize
    if reader == "direct" and info["direct"]:
        # pinned slabs cannot take the storage DMA: the reads go through the bounce buffers
        assert info["bytes_bounced"] > 0 and info["bytes_buffered"] == 0
    else:
        assert info["bytes_direct"] == info["bytes_bounced"] == 0
    assert sum(m.evictions for m in rt.telemetry.history) > 0
    rt.shutdown()


@pytest.mark.gpu
@pytest.mark.parametrize("reader", ["mmap", "pread", "direct"])
def test_sharded_files_and_pinned_images(tmp_path, reader):
    """One shard per block (the bench's config-3 layout) and pinned source images: the first load
    reads the file ranges into the image, later loads DMA from it."""
    from safetensors.torch import save_file

    import stagehand_amd as stagehand
    from tests.streaming_models import TinyStack, init_

    model = init_(TinyStack(n=4, hidden=128, mlp=4)).to(torch.bfloat16)
    ref = init_(TinyStack(n=4, hidden=128, mlp=4)).to(device="cuda", dtype=torch.bfloat16)
    shards = tmp_path / "shards"
    shards.mkdir()
    weight_map = {}
    for i, blk in enumerate(model.blocks):
        tensors = {f"blocks.{i}.{k}": v.detach().contiguous() for k, v in blk.named_parameters()}
        save_file(tensors, str(shards / f"blocks.{i}.safetensors"))
        weight_map.update({k: f"blocks.{i}.safetensors" for k in tensors})
    (shards / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    model.requires_grad_(False)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(file_reader=reader, pinned_source_cache=True, vram_high_watermark_mb=int(base_mb) + 1,
                  vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_file_backed_sharded(str(shards)) > 0
    x = torch.randn(3, 128).to(torch.bfloat16).cuda()
    outs = []
    for step in range(3):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            outs.append(model(x))
        rt.end_step()
    with torch.no_grad():
        want = ref(x)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    assert rt.engine.pinned_image_bytes > 0
    if reader != "mmap":
        files = rt.scheduler._weight_files.files()
        assert len(files) == 4
        # each file was read once, into its image
        for f in files:
            info = f.info()
            assert info["bytes_direct"] + info["bytes_bounced"] + info["bytes_buffered"] <= f.size
    rt.shutdown()


@pytest.mark.gpu
@pytest.mark.parametrize("reader", ["mmap", "pread", "direct"])
def test_pinned_images_survive_module_params_changing_dtype(tmp_path, reader):
    """Norm weights missing from the file stay in the module as fp32 and come back from the
    first eviction as bf16. The block's source must keep its layout across that change, so each
    pinned source image is filled once and every later load DMAs from it."""
    from safetensors.torch import save_file

    import stagehand_amd as stagehand
    from tests.streaming_models import TinyStack, init_

    model = init_(TinyStack(n=4, hidden=128, mlp=4))  # fp32
    save_file({k: v.detach().to(torch.bfloat16).contiguous() for k, v in model.state_dict().items()
               if ".norm." not in k}, str(tmp_path / "w.safetensors"))
    ref = init_(TinyStack(n=4, hidden=128, mlp=4)).to(device="cuda", dtype=torch.bfloat16)
    model.requires_grad_(False)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(file_reader=reader, pinned_source_cache=True, vram_high_watermark_mb=int(base_mb) + 1,
                  vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    rt.convert_registry_to_file_backed(str(tmp_path / "w.safetensors"))
    x = torch.randn(3, 128).to(torch.bfloat16).cuda()
    images = None
    for step in range(3):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            y = model(x)
        rt.end_step()
        with torch.no_grad():
            want = ref(x)
        torch.cuda.synchronize()
        assert torch.equal(_bits(y), _bits(want)), step
        keys = {b: v[0] for b, v in rt.engine._images.items()}
        if images is not None:
            assert keys == images, f"step {step}: a block's source layout changed"
        images = keys
    assert len(images) == 4
    assert sum(m.evictions for m in rt.telemetry.history) > 0
    if reader != "mmap":
        (f,) = rt.scheduler._weight_files.files()
        info = f.info()
        assert info["bytes_direct"] + info["bytes_bounced"] + info["bytes_buffered"] <= f.size
    rt.shutdown()


@pytest.mark.gpu
@pytest.mark.parametrize("reader", ["mmap", "pread", "direct"])
@pytest.mark.parametrize("padded,with_zp", [(0, False), (16, True)])
def test_squareq_v2_streaming_per_reader(tmp_path, reader, padded, with_zp):
    """A SquareQ V2 slab (safetensors + manifest) streamed with each reader gives the host dequant
    of src/stagehand/scheduler.py:285-308 bit for bit; with the native readers the int8 rows,
    scales and zero points are read from the file straight into the pinned slab."""
    import stagehand_amd as stagehand
    from stagehand_amd.squareq_v2 import write_v2_slab
    from tests.streaming_models import TinyStack, expected_squareq_weight, init_, squareq_payload

    model = init_(TinyStack(n=4, hidden=96, mlp=4))
    payload = squareq_payload(model, padded=padded, with_zp=with_zp)
    layers = {}
    for name, L in payload["layers"].items():
        t = {"qweight": L["qweight"], "scale": L["scale"], "bias": L["bias"], "in_features": L["qweight"].shape[1] - padded}
        if with_zp:
            t["zero_point"] = L["zero_point"]
        layers[name] = t
    path = tmp_path / "tiny.safetensors"
    manifest = write_v2_slab(str(path), layers)
    model.requires_grad_(False)
    ref = init_(TinyStack(n=4, hidden=96, mlp=4))
    for bi, blk in enumerate(ref.blocks):
        for lname in ("fc1", "fc2"):
            lin = getattr(blk, lname)
            L = payload["layers"][f"blocks.{bi}.{lname}"]
            with torch.no_grad():
                lin.weight.copy_(expected_squareq_weight(L, *lin.weight.shape, torch.bfloat16).float())
                lin.bias.copy_(L["bias"].to(torch.bfloat16).float())
    ref = ref.to(device="cuda", dtype=torch.bfloat16)
    model = model.to(torch.bfloat16)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(file_reader=reader, vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb),
                  prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_squareq_v2_backed(str(path), manifest) == 4 * 4
    x = torch.randn(5, 96).to(torch.bfloat16).cuda()
    outs = []
    for step in range(3):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            outs.append(model(x))
        rt.end_step()
    with torch.no_grad():
        want = ref(x)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    assert sum(m.evictions for m in rt.telemetry.history) > 0
    if reader != "mmap":
        (f,) = rt.scheduler._weight_files.files()
        info = f.info()
        read = info["bytes_direct"] + info["bytes_bounced"] + info["bytes_buffered"]
        int8 = sum(L["qweight"].numel() - padded * L["qweight"].shape[0] for L in payload["layers"].values())
        assert read >= int8  # every step's int8 rows came through the reader
        assert not rt.scheduler._squareq_layers  # no host views of the slab were made
    rt.shutdown()


def test_builder_rejects_inconsistent_file_ranges(tmp_path):
    path = tmp_path / "x.bin"
    np.zeros(4096, dtype=np.uint8).tofile(path)
    f = WeightFile(path)
    b = SourceBuilder(torch.bfloat16, 4096)
    with pytest.raises(ValueError, match="does not hold"):
        b.add_file_param(0, FileRange(f, 0, 100), torch.bfloat16, 64)
    with pytest.raises(ValueError, match="not 4 rows"):
        b.add_dequant_file(0, FileRange(f, 0, 100), 4, 32, 32, FileRange(f, 0, 16), None)
    with pytest.raises(ValueError, match="shorter than"):
        b.add_dequant_file(0, FileRange(f, 0, 128), 4, 32, 33, FileRange(f, 0, 16), None)
    with pytest.raises(ValueError, match="scale range"):
        b.add_dequant_file(0, FileRange(f, 0, 128), 4, 32, 32, FileRange(f, 0, 12), None)
    with pytest.raises(ValueError, match="zero point range"):
        b.add_dequant_file(0, FileRange(f, 0, 128), 4, 32, 32, FileRange(f, 0, 16), FileRange(f, 0, 8))
    f.close()


@pytest.mark.gpu
def test_load_errors_are_reported_and_finish_the_load(tmp_path):
    """A range past the end of its file is refused at submit (ValueError); a file that shrinks
    after it was opened fails the load with the read error (TransferError), and the failed load
    is finished: later waits and shutdown do not raise it again."""
    from stagehand_amd.errors import TransferError
    from stagehand_amd.pool import PinnedPool
    from stagehand_amd.transfer import AsyncTransferEngine, BlockSource

    path = tmp_path / "w.bin"
    data = np.random.default_rng(1).integers(0, 256, size=3 << 20, dtype=np.uint8)
    data.tofile(path)
    f = WeightFile(path)
    pool = PinnedPool(total_mb=8, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool)
    dst = torch.empty(2 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="past the end"):
        eng.submit_block_load("b", BlockSource([(0, FileRange(f, data.size - 8, 16))], 16), dst)
    h = eng.submit_block_load("ok", BlockSource([(0, FileRange(f, 4096, 2 << 20))], 2 << 20), dst)
    eng.wait(h)
    assert np.array_equal(dst.cpu().numpy(), data[4096:4096 + (2 << 20)])
    with open(path, "r+b") as fh:
        fh.truncate(1 << 20)
    h = eng.submit_block_load("short", BlockSource([(0, FileRange(f, 0, 2 << 20))], 2 << 20), dst)
    with pytest.raises(TransferError, match="unexpected end of file"):
        eng.wait(h)
    eng.wait(h)  # finished: no second error
    assert eng.inflight_count() == 0
    eng.shutdown()
    pool.shutdown()
    f.close()
