"""VMM residency allocator (stagehand_amd.vmm over sh_vmm_* in the C ABI).

The GPU cases restate the reference's own expectations for the allocator
(vmm_tests/integration.rs:27-225: slab/region lifecycle, mapping, eviction
under a ceiling by priority, watermark refusal and promotion, refcount
protection, prefetch, stats) and its Python surface (vmm_tests/python_test.py:
11-132: DLPack tensors, handle release, MemoryError on a watermark, tensors
outliving their handle, compute on mapped memory), then run a streamed block
model through StagehandRuntime's VMM path against the same model unstreamed.
"""
from __future__ import annotations

import time

import pytest
import torch

from stagehand_amd import vmm
from stagehand_amd.vmm import RegionState, SlabAllocator


def test_unavailable_without_device():
    if torch.cuda.is_available():
        pytest.skip("device present")
    assert vmm.is_available() is False


gpu = pytest.mark.gpu


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@gpu
def test_slab_and_region_lifecycle():
    a = SlabAllocator(device=0)
    g = a.granularity()
    assert g > 0 and a.stats()["vram_ceiling"] > 0
    slab = a.create_slab(g * 10)
    assert [a.define_region(slab, i * g, g) for i in range(10)] == list(range(10))
    with pytest.raises(ValueError):
        a.define_region(slab, g // 2, g)  # not a granularity multiple
    with pytest.raises(ValueError):
        a.define_region(slab, 10 * g, g)  # past the end of the slab
    with pytest.raises(ValueError):
        a.define_region(slab + 7, 0, g)
    s = a.stats()
    assert (s["total_slabs"], s["total_regions"], s["mapped_bytes"]) == (1, 10, 0)
    a.destroy_slab(slab)
    with pytest.raises(ValueError):
        a.destroy_slab(slab)
    a.close()


@gpu
def test_ensure_resident_maps_and_keeps_data():
    a = SlabAllocator(device=0)
    g = a.granularity()
    slab = a.create_slab(g)
    r = a.define_region(slab, 0, g)
    h = a.ensure_resident(slab, r, _stream())
    assert h.data_ptr() != 0
    st = a.region_stats(slab, r)
    assert st["state"] == RegionState.RESIDENT and st["refcount"] == 1
    assert a.stats()["mapped_bytes"] >= g
    t = h.as_tensor("int32", [g // 4])
    t.copy_(torch.arange(g // 4, dtype=torch.int32, device="cuda"))
    gen = h.generation()
    del t
    h.release()
    assert a.region_stats(slab, r)["refcount"] == 0
    h2 = a.ensure_resident(slab, r, _stream())  # fast path: still mapped, data kept
    assert h2.generation() == gen
    assert torch.equal(h2.as_tensor("int32", [g // 4]).cpu(), torch.arange(g // 4, dtype=torch.int32))
    h2.release()
    a.destroy_slab(slab)
    a.close()


@gpu
def test_eviction_under_pressure_by_priority():
    a = SlabAllocator(device=0)
    g = a.granularity()
    a.set_vram_ceiling(2 * g)
    s1 = a.create_slab(2 * g)
    r1a, r1b = a.define_region(s1, 0, g), a.define_region(s1, g, g)
    # a slab's watermark starts at its first region count (allocator.rs:193-195), so
    # region 1 opens only with the slab's promotion (the reference's own test maps it
    # without one, vmm_tests/integration.rs:91-93, which its allocator refuses)
    with pytest.raises(MemoryError):
        a.ensure_resident(s1, r1b, _stream())
    a.set_priority(s1, 5)
    s2 = a.create_slab(g)
    r2 = a.define_region(s2, 0, g)
    h1a = a.ensure_resident(s1, r1a, _stream())
    h1b = a.ensure_resident(s1, r1b, _stream())
    gen1a = h1a.generation()
    h1a.release()
    h1b.release()
    a.set_priority(s2, 10)
    h2 = a.ensure_resident(s2, r2, _stream())  # evicts the oldest region of the low-priority slab
    assert h2.data_ptr() != 0
    assert a.region_stats(s1, r1a)["state"] == RegionState.UNMAPPED
    assert a.region_stats(s1, r1b)["state"] == RegionState.RESIDENT
    assert a.region_stats(s1, r1a)["watermark"] == r1a  # lowered to the evicted region
    assert a.stats()["mapped_bytes"] == 2 * g
    h2.release()
    a.set_priority(s1, 20)  # re-opens slab 1
    h = a.ensure_resident(s1, r1a, _stream())
    assert h.generation() != gen1a  # a new mapping: contents are gone
    h.release()
    a.destroy_slab(s2)
    a.destroy_slab(s1)
    a.close()


@gpu
def test_watermark_refusal_and_promotion():
    a = SlabAllocator(device=0)
    g = a.granularity()
    a.set_vram_ceiling(g)
    s1 = a.create_slab(g)
    r1 = a.define_region(s1, 0, g)
    s2 = a.create_slab(2 * g)
    r2a = a.define_region(s2, 0, g)
    a.define_region(s2, g, g)
    h1 = a.ensure_resident(s1, r1, _stream())
    with pytest.raises(MemoryError):
        a.ensure_resident(s2, r2a, _stream())
    with pytest.raises(MemoryError):  # slab 2 is watermarked now
        a.ensure_resident(s2, r2a, _stream())
    h1.release()
    a.set_priority(s2, 10)
    h2 = a.ensure_resident(s2, r2a, _stream())
    assert h2.data_ptr() != 0
    h2.release()
    a.destroy_slab(s1)
    a.destroy_slab(s2)
    a.close()


@gpu
def test_refcount_prevents_eviction_and_slab_destroy():
    a = SlabAllocator(device=0)
    g = a.granularity()
    a.set_vram_ceiling(g)
    s = a.create_slab(2 * g)
    r1, r2 = a.define_region(s, 0, g), a.define_region(s, g, g)
    a.set_priority(s, 1)  # open both regions
    h1 = a.ensure_resident(s, r1, _stream())
    with pytest.raises(MemoryError):  # r1 is held: nothing to evict
        a.ensure_resident(s, r2, _stream())
    with pytest.raises(RuntimeError, match="active handles"):
        a.destroy_slab(s)
    h1.release()
    a.set_priority(s, 2)  # the refused map lowered the watermark; promotion re-opens it
    h2 = a.ensure_resident(s, r2, _stream())
    assert a.region_stats(s, r1)["state"] == RegionState.UNMAPPED
    h2.release()
    a.destroy_slab(s)
    a.close()


@gpu
def test_prefetch_maps_on_the_worker():
    a = SlabAllocator(device=0)
    g = a.granularity()
    s = a.create_slab(g)
    r = a.define_region(s, 0, g)
    a.prefetch(s, r)
    deadline = time.monotonic() + 5.0
    while a.region_stats(s, r)["state"] != RegionState.RESIDENT and time.monotonic() < deadline:
        time.sleep(0.005)
    assert a.region_stats(s, r)["state"] == RegionState.RESIDENT
    h = a.ensure_resident(s, r, _stream())
    assert h.data_ptr() != 0
    h.release()
    a.destroy_slab(s)
    a.close()


@gpu
def test_tensors_release_and_compute():
    a = SlabAllocator(device=0)
    mib = 1 << 20
    s = a.create_slab(64 * mib)
    r = a.define_region(s, 0, 32 * mib)
    a.set_priority(s, 100)
    h = a.ensure_resident(s, r, _stream())
    t = h.as_tensor("bfloat16", [16 * mib])
    assert t.device.type == "cuda" and t.dtype == torch.bfloat16 and t.shape == (16 * mib,)
    with pytest.raises(ValueError):
        h.as_tensor("complex64", [4])
    with pytest.raises(ValueError):
        h.as_tensor("float32", [64 * mib])  # larger than the region
    f = h.as_tensor("float32", [1024, 256])
    f.copy_(torch.randn(1024, 256, device="cuda"))
    w = torch.randn(256, 512, device="cuda")
    assert torch.allclose(torch.matmul(f, w), torch.matmul(f.clone(), w))
    h.release()
    with pytest.raises(RuntimeError):
        h.as_tensor("float32", [1024])
    with pytest.raises(RuntimeError):
        h.release()
    assert a.region_stats(s, r)["refcount"] == 2  # the tensors t and f hold their own references
    assert (f + 1).shape == (1024, 256)
    del t, f
    torch.cuda.synchronize()
    assert a.region_stats(s, r)["refcount"] == 0
    a.destroy_slab(s)
    a.close()


@gpu
def test_numpy_integers_for_ids_stream_and_shape():
    """The binding's fast path passes Python ints straight to the C ABI; numpy integers (ids kept
    in arrays, a shape from ``ndarray.shape`` arithmetic) take the converting path."""
    import numpy as np

    a = SlabAllocator(device=0)
    mib = 1 << 20
    s = a.create_slab(8 * mib)
    r = a.define_region(s, 0, 4 * mib)
    a.set_priority(s, 100)
    h = a.ensure_resident(np.uint32(s), np.int64(r), np.int64(_stream()))
    t = h.as_tensor("float32", [np.int64(512), np.int32(2048)])
    assert t.shape == (512, 2048)
    t.fill_(3.0)
    assert float(t.sum()) == 3.0 * 512 * 2048
    del t
    h.release()
    torch.cuda.synchronize()
    a.destroy_slab(s)
    a.close()


@gpu
@pytest.mark.parametrize("reader", ["pread", "mmap"])
@pytest.mark.parametrize("mode", ["roomy", "tight", "tight_reopen"])
def test_runtime_serves_blocks_from_vmm(tmp_path, mode, reader):
    """A file-backed model registered with the VMM backend gives the unstreamed outputs.
    With a ceiling of two blocks the first eviction lowers the model slab's watermark and
    later blocks take the block-swap path (the parameters it holds in the module, such as
    the norms, must survive the VMM blocks); re-activating the model every step re-opens
    the slab, so blocks are evicted, re-mapped and re-filled from the file — by the native
    reader or through mappings."""
    tight = mode != "roomy"
    import stagehand_amd as stagehand
    from tests.streaming_models import TinyStack, init_, save_safetensors

    model = init_(TinyStack(n=6, hidden=256, mlp=4)).to(torch.bfloat16)
    path = tmp_path / "w.safetensors"
    save_safetensors(model, path, torch.bfloat16)
    ref = init_(TinyStack(n=6, hidden=256, mlp=4)).to(device="cuda", dtype=torch.bfloat16)
    model.requires_grad_(False)
    cfg = stagehand.StagehandConfig(pinned_pool_mb=64, pinned_slab_mb=4, vram_high_watermark_mb=200000,
                                    vram_low_watermark_mb=100000, prefetch_window_blocks=2, nan_inf_check=False,
                                    strict_bf16=False, telemetry_enabled=False, file_reader=reader)
    cfg.telemetry_file = None
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    rt.convert_registry_to_file_backed(str(path))
    assert rt.vmm is not None
    handle = rt.vmm_register_model("tiny", "bfloat16", str(path))
    if tight:
        g = rt.vmm.allocator.granularity()
        rt.vmm.set_ceiling(2 * -(-max(handle.block_sizes) // g) * g)
    x = torch.randn(4, 256).to(torch.bfloat16).cuda()
    for step in range(3):
        if mode == "tight_reopen":
            rt.vmm.activate_model("tiny")
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            y = model(x)
        rt.end_step()
        with torch.no_grad():
            yr = ref(x)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), yr.view(torch.int16)), step
    stats = rt.vmm.stats()
    if tight:
        assert stats["mapped_bytes"] <= 2 * g * -(-max(handle.block_sizes) // g)
        assert stats["evictions"] >= 1
    if mode == "tight_reopen":
        # some block was evicted, mapped again and re-filled (its mapping generation is 2 or more)
        assert max(g for g in handle._filled_generation if g is not None) >= 2
    assert stats["unmap_failures"] == 0
    assert not rt._vmm_active_blocks
    if not tight:
        assert handle.fills_ahead >= 5  # the first step filled every block after the first ahead of its use
    assert not handle._pending_fills
    if reader == "pread":
        read = sum(f.info()["bytes_buffered"] for f in handle._weight_files.values())
        filled = sum(size for size, g in zip(handle.block_sizes, handle._filled_generation) if g is not None)
        assert read >= filled > 0  # the blocks served from the VMM were filled by the native reader
    rt.shutdown()
