"""End-to-end parity of the device streaming path (native loader + unpack kernels).

Every case compares device results with the reference's host computation
(the torch CPU ops of src/stagehand/scheduler.py) bit for bit: streamed
parameter bytes, and block outputs against the same model run unstreamed.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import stagehand_amd as stagehand
from stagehand_amd.config import StagehandConfig
from tests.streaming_models import TinyStack, expected_squareq_weight, init_, save_safetensors, squareq_payload

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32).cpu()


def _config(**kw) -> StagehandConfig:
    base = dict(pinned_pool_mb=64, pinned_slab_mb=4, vram_high_watermark_mb=200000, vram_low_watermark_mb=100000,
                prefetch_window_blocks=2, telemetry_enabled=True, telemetry_file=None, nan_inf_check=False,
                strict_bf16=False)
    base.update(kw)
    cfg = StagehandConfig(**{k: v for k, v in base.items() if k != "telemetry_file"})
    cfg.telemetry_file = None
    return cfg


def _run_blocks(rt, model, x, steps=2):
    outs = []
    for step in range(steps):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            outs.append(model(x))
        rt.end_step()
    torch.cuda.synchronize()
    return outs


def test_config1_layer_mode_bytes_and_outputs():
    """8 x Linear(4096, 4096) fp32, dtype bf16, prefetch_k=3: trace step then scheduled step."""
    torch.manual_seed(0)
    model = torch.nn.Sequential(*[torch.nn.Linear(4096, 4096) for _ in range(8)])
    with torch.no_grad():
        for m in model:
            m.weight.normal_(0, 0.02)
            m.bias.zero_()
    ref = torch.nn.Sequential(*[torch.nn.Linear(4096, 4096) for _ in range(8)])
    ref.load_state_dict(model.state_dict())
    want_bytes = [torch.cat([m.weight.detach().to(torch.bfloat16).reshape(-1), m.bias.detach().to(torch.bfloat16)]) for m in ref]
    ref = ref.to(device="cuda", dtype=torch.bfloat16)
    x = torch.randn(16, 4096).to(torch.bfloat16).cuda()
    m = stagehand.layer(model, dtype=torch.bfloat16, prefetch_k=3, inference_mode=True)
    rt = m._stagehand_layer_runtime
    assert (rt.config.pinned_slab_mb, rt.pool.num_slabs) == (64, 7)
    with torch.no_grad():
        y0 = m(x)
        y1 = m(x)
        yr = ref(x)
    torch.cuda.synchronize()
    assert rt.mode == "scheduled"
    assert torch.equal(_bits(y0), _bits(y1))
    assert torch.equal(_bits(y0), _bits(yr))
    for i, layer in enumerate(model):
        entry = rt.residency.get_entry(str(i))
        assert entry.gpu_tensor is not None
        got = entry.gpu_tensor.view(torch.bfloat16)
        assert got.numel() * 2 == 33_562_624
        assert torch.equal(_bits(got), _bits(want_bytes[i]))
    rt.shutdown()


@pytest.mark.parametrize("padded,with_zp", [(0, False), (16, True), (3, False)])
def test_squareq_block_mode_matches_host_dequant(tmp_path, padded, with_zp):
    model = init_(TinyStack(n=5, hidden=96, mlp=4))
    payload = squareq_payload(model, padded=padded, with_zp=with_zp)
    path = tmp_path / "tiny.fpk"
    torch.save(payload, path)
    for p in model.parameters():
        p.requires_grad_(False)
    ref = init_(TinyStack(n=5, hidden=96, mlp=4))
    for bi, blk in enumerate(ref.blocks):
        for lname in ("fc1", "fc2"):
            lin = getattr(blk, lname)
            layer = payload["layers"][f"blocks.{bi}.{lname}"]
            with torch.no_grad():
                lin.weight.copy_(expected_squareq_weight(layer, *lin.weight.shape, torch.bfloat16).float())
                lin.bias.copy_(layer["bias"].to(torch.bfloat16).float())
    ref = ref.to(device="cuda", dtype=torch.bfloat16)
    model = model.to(torch.bfloat16)
    rt = stagehand.StagehandRuntime(model, _config(), block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    n = rt.convert_registry_to_file_backed(str(path))
    assert n == 5 * 4
    x = torch.randn(7, 96).to(torch.bfloat16).cuda()
    outs = _run_blocks(rt, model, x, steps=2)
    with torch.no_grad():
        want = ref(x)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    # the streamed buffer of a resident block holds exactly the host dequant bytes
    for bi in range(5):
        e = rt.residency.get_entry(f"blocks.{bi}")
        if e.gpu_tensor is None:
            continue
        blk = model.blocks[bi]
        for lname in ("fc1", "fc2"):
            lin = getattr(blk, lname)
            layer = payload["layers"][f"blocks.{bi}.{lname}"]
            assert torch.equal(_bits(lin.weight), _bits(expected_squareq_weight(layer, *lin.weight.shape, torch.bfloat16)))
    m0 = rt.telemetry.history[0]
    assert m0.h2d_bytes == sum(rt.registry.get(f"blocks.{i}").size_bytes for i in range(5))
    rt.shutdown()


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_file_backed_block_mode(tmp_path, src_dtype):
    model = init_(TinyStack(n=6, hidden=64, mlp=4))
    path = tmp_path / "tiny.safetensors"
    save_safetensors(model, path, src_dtype)
    ref = init_(TinyStack(n=6, hidden=64, mlp=4)).to(device="cuda", dtype=torch.bfloat16)
    for p in model.parameters():
        p.requires_grad_(False)
    model = model.to(torch.bfloat16)
    rt = stagehand.StagehandRuntime(model, _config(), block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=True)
    assert rt.convert_registry_to_file_backed(str(path)) == 6 * 4
    x = torch.randn(5, 64).to(torch.bfloat16).cuda()
    outs = _run_blocks(rt, model, x, steps=3)
    with torch.no_grad():
        want = ref(x)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    rt.shutdown()


def test_eviction_under_tight_watermarks_preserves_values(tmp_path):
    """Blocks are evicted and reloaded every step (watermarks below one block) and results stay exact."""
    model = init_(TinyStack(n=8, hidden=128, mlp=4))
    path = tmp_path / "tiny.fpk"
    payload = squareq_payload(model)
    torch.save(payload, path)
    for p in model.parameters():
        p.requires_grad_(False)
    model = model.to(torch.bfloat16)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16, inference_mode=True)
    rt.convert_registry_to_file_backed(str(path))
    x = torch.randn(3, 128).to(torch.bfloat16).cuda()
    outs = _run_blocks(rt, model, x, steps=3)
    assert all(torch.equal(_bits(o), _bits(outs[0])) for o in outs)
    hist = rt.telemetry.history
    assert sum(m.evictions for m in hist) > 0
    assert hist[0].h2d_bytes == sum(rt.registry.get(f"blocks.{i}").size_bytes for i in range(8))
    assert all(m.h2d_bytes > 0 for m in hist[1:])
    rt.shutdown()


def test_module_backed_training_round_trip():
    """Training (save-back) eviction keeps updated values; matches an unstreamed run."""
    torch.manual_seed(3)
    model = init_(TinyStack(n=4, hidden=64, mlp=2)).to(torch.bfloat16)
    ref = init_(TinyStack(n=4, hidden=64, mlp=2)).to(device="cuda", dtype=torch.bfloat16)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16, inference_mode=False)
    # activations entering the blocks carry grad (as they do after an embedding),
    # so each block's full backward hook fires after its own backward ops
    x = torch.randn(4, 64).to(torch.bfloat16).cuda().requires_grad_()
    rt.begin_step(0)
    with rt.managed_forward(), rt.managed_backward():
        y = model(x)
        y.float().square().mean().backward()
    rt.end_step()
    yr = ref(x)
    yr.float().square().mean().backward()
    torch.cuda.synchronize()
    assert torch.equal(_bits(y), _bits(yr))
    for (n1, p1), (n2, p2) in zip(model.named_parameters(), ref.named_parameters()):
        assert p1.grad is not None, n1
        assert torch.allclose(p1.grad.float().cpu(), p2.grad.float().cpu(), atol=1e-3, rtol=1e-2), n1
    rt.shutdown()


def test_dit_squareq_streaming_matches_unstreamed(tmp_path):
    """A small Flux-style DiT built on the meta device, SquareQ-backed, streamed in block
    mode, equals the same DiT run unstreamed with the host-dequantised weights."""
    import sys
    from pathlib import Path as _P

    sys.path.insert(0, str(_P(__file__).resolve().parent.parent))
    from bench_workloads import write_dit_squareq
    from bench_workloads import DIT_BLOCK_PATTERN, FluxStyleDiT, dit_linear_layers, materialize_norms_

    kw = dict(depth_double=2, depth_single=3, hidden=256, heads=2, mlp_ratio=4.0)
    with torch.device("meta"):
        model = FluxStyleDiT(**kw)
    model.requires_grad_(False)
    materialize_norms_(model)
    path = tmp_path / "dit.fpk"
    layers = write_dit_squareq(model, path, seed=5)

    ref = FluxStyleDiT(**kw)
    with torch.no_grad():
        for name, lin in dit_linear_layers(ref):
            L = layers[name]
            lin.weight.copy_(expected_squareq_weight(L, lin.out_features, lin.in_features, torch.bfloat16).float())
            lin.bias.copy_(L["bias"].float())
        for mod in ref.modules():
            if isinstance(mod, torch.nn.RMSNorm):
                mod.weight.fill_(1.0)
    ref = ref.to(device="cuda", dtype=torch.bfloat16)

    cfg = _config(pinned_pool_mb=16, pinned_slab_mb=1, prefetch_window_blocks=2, max_inflight_transfers=3)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=DIT_BLOCK_PATTERN, dtype=torch.bfloat16, inference_mode=True)
    assert rt.convert_registry_to_file_backed(str(path)) == 2 * 20 + 3 * 6
    g = torch.Generator(device="cuda").manual_seed(0)
    img = torch.randn(1, 64, 256, device="cuda", generator=g).to(torch.bfloat16)
    txt = torch.randn(1, 16, 256, device="cuda", generator=g).to(torch.bfloat16)
    vec = torch.randn(1, 256, device="cuda", generator=g).to(torch.bfloat16)
    outs = []
    for step in range(2):
        rt.begin_step(step)
        with torch.no_grad(), rt.managed_forward():
            outs.append(model(img, txt, vec))
        rt.end_step()
    with torch.no_grad():
        want = ref(img, txt, vec)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(_bits(y), _bits(want))
    # PCIe bytes: int8 weights + fp32 scales + bf16 biases/norms, about half the bf16 block bytes
    sent = rt.engine.bytes_h2d
    bf16 = sum(e.size_bytes for e in rt.registry.blocks_in_order())
    assert sent < 0.6 * 2 * bf16
    rt.shutdown()


def test_pinned_source_images_refresh_mutable_params(tmp_path):
    """With pinned source images, later loads DMA from the image; module-backed
    (mutable) parameters are re-gathered, so changes to them are streamed."""
    model = init_(TinyStack(n=4, hidden=64, mlp=4))
    payload = squareq_payload(model)
    path = tmp_path / "tiny.fpk"
    torch.save(payload, path)
    for p in model.parameters():
        p.requires_grad_(False)
    model = model.to(torch.bfloat16)
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1,
                  pinned_source_cache=True)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16, inference_mode=True)
    rt.convert_registry_to_file_backed(str(path))
    x = torch.randn(3, 64).to(torch.bfloat16).cuda()
    y0 = _run_blocks(rt, model, x, steps=2)
    assert torch.equal(_bits(y0[0]), _bits(y0[1]))
    assert rt.engine.pinned_image_bytes > 0
    # change block 0's norm weight (module-backed) while the block is evicted to CPU
    e0 = rt.residency.get_entry("blocks.0")
    if e0.gpu_tensor is not None:
        rt.scheduler._evict_block("blocks.0")
    with torch.no_grad():
        model.blocks[0].norm.weight.mul_(2.0)
    y1 = _run_blocks(rt, model, x, steps=1)[0]
    assert not torch.equal(_bits(y1), _bits(y0[0]))
    rt.shutdown()
    # reference: an identical model with the same change, streamed through the staged (non-pinned) path
    model2 = init_(TinyStack(n=4, hidden=64, mlp=4))
    for p in model2.parameters():
        p.requires_grad_(False)
    model2 = model2.to(torch.bfloat16)
    with torch.no_grad():
        model2.blocks[0].norm.weight.mul_(2.0)
    rt2 = stagehand.StagehandRuntime(model2, _config(), block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                     inference_mode=True)
    rt2.convert_registry_to_file_backed(str(path))
    y2 = _run_blocks(rt2, model2, x, steps=1)[0]
    assert torch.equal(_bits(y1), _bits(y2))
    rt2.shutdown()


def _train_dit(seed: int):
    from bench_workloads import TrainDiT, init_train_dit_

    return init_train_dit_(TrainDiT(depth=4, hidden=128, heads=4, mlp_ratio=2.0, rank=8), seed)


@pytest.mark.parametrize("frozen_host_copies,save_back,changed_chunks",
                         [(False, "sdma", False), (False, "sdma", True), (True, "sdma", False), (False, "stream", False)])
def test_checkpointed_lora_training_round_trip(frozen_host_copies, save_back, changed_chunks):
    """Config-5 shape in small: frozen base weights, trainable LoRA, activation checkpointing
    (blocks recomputed in backward under the runtime's hooks), module-backed eviction every
    block, an SGD step on the LoRA parameters between steps. Outputs, LoRA gradients and the
    updated LoRA weights match the same model trained unstreamed: bit for bit at step 0, within
    tolerance after SGD steps (an evicted block's LoRA update runs on the host, a resident one's
    on the device, and the two round the bf16 update differently); with frozen host copies the
    frozen weights are not copied back at eviction; with changed-chunk save-backs only the first
    save-back of a block copies all of it. Save-backs on the SDMA engine and on the copy stream."""
    from bench_workloads import TRAIN_BLOCK_PATTERN

    model = _train_dit(5)
    ref = _train_dit(5).cuda()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 32, 128, generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn(1, 16, 128, generator=g).to(torch.bfloat16).cuda()
    vec = torch.randn(1, 128, generator=g).to(torch.bfloat16).cuda()
    target = torch.randn(1, 32, 128, generator=g).cuda()
    base_mb = torch.cuda.memory_allocated() / 2**20
    cfg = _config(vram_high_watermark_mb=int(base_mb) + 1, vram_low_watermark_mb=int(base_mb), prefetch_window_blocks=1,
                  frozen_host_copies=frozen_host_copies, save_back_engine=save_back,
                  save_back_changed_chunks=changed_chunks, save_back_chunk_bytes=4096)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=TRAIN_BLOCK_PATTERN, dtype=torch.bfloat16,
                                    inference_mode=False)
    lora = [p for n, p in model.named_parameters() if "lora" in n]
    lora_ref = [p for n, p in ref.named_parameters() if "lora" in n]
    opt = torch.optim.SGD(lora, lr=0.5, foreach=False)
    opt_ref = torch.optim.SGD(lora_ref, lr=0.5, foreach=False)
    for step in range(3):
        xi = x.clone().requires_grad_()
        rt.begin_step(step)
        with rt.managed_forward(), rt.managed_backward():
            y = model(xi, ctx, vec)
            torch.nn.functional.mse_loss(y.float(), target).backward()
        rt.end_step()
        xr = x.clone().requires_grad_()
        yr = ref(xr, ctx, vec)
        torch.nn.functional.mse_loss(yr.float(), target).backward()
        torch.cuda.synchronize()
        if step == 0:
            # Before any optimizer step both models hold the same bf16 weights and run the same
            # kernels on them: outputs and LoRA gradients are bit-identical.
            assert torch.equal(y, yr), "step 0 outputs differ from the unstreamed model"
        assert torch.allclose(y.float(), yr.float(), atol=2e-2, rtol=2e-2), step
        for (n, p), q in zip([(n, p) for n, p in model.named_parameters() if "lora" in n], lora_ref):
            assert p.grad is not None, n
            if step == 0:
                assert torch.equal(p.grad.cpu(), q.grad.cpu()), (step, n)
            assert torch.allclose(p.grad.float().cpu(), q.grad.float().cpu(), atol=1e-3, rtol=5e-2), (step, n)
        opt.step()
        opt_ref.step()
        opt.zero_grad(set_to_none=True)
        opt_ref.zero_grad(set_to_none=True)
    for (n, p), q in zip([(n, p) for n, p in model.named_parameters() if "lora" in n], lora_ref):
        assert torch.allclose(p.float().cpu(), q.float().cpu(), atol=1e-2, rtol=5e-2), n
    # every eviction of a block copies back its LoRA weights and gradients; without
    # frozen host copies also its frozen weights
    evictions = sum(m.evictions for m in rt.telemetry.history)
    blk = ref.blocks[0]
    frozen_per_block = sum(p.numel() * 2 for n, p in blk.named_parameters() if "lora" not in n)
    lora_per_block = sum(p.numel() * 2 for n, p in blk.named_parameters() if "lora" in n)
    sent_back = rt.engine.bytes_d2h
    assert evictions > 0
    if frozen_host_copies:
        assert sent_back <= evictions * 2 * lora_per_block
    elif changed_chunks:
        assert rt.engine.bytes_d2h_requested > 0
        assert sent_back < evictions * frozen_per_block
    else:
        assert sent_back >= evictions * frozen_per_block
    rt.shutdown()


class _SimpleMLP(torch.nn.Module):
    def __init__(self, hidden: int = 16, num_layers: int = 3) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList(torch.nn.Linear(hidden, hidden, bias=False) for _ in range(num_layers))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x)
        return x


@pytest.mark.parametrize("inference_mode", [False, True])
def test_layer_mode_fp32_matches_unwrapped(inference_mode):
    """Layer mode with fp32 storage gives the unwrapped model's outputs on the trace step, the
    scheduled step and later steps, and gradients on every managed parameter (the checks of the
    reference's tests/test_compat_ramtorch.py:263-340, through stagehand.layer)."""
    torch.manual_seed(3)
    model = _SimpleMLP(hidden=64, num_layers=4)
    ref = _SimpleMLP(hidden=64, num_layers=4)
    ref.load_state_dict(model.state_dict())
    ref = ref.cuda()
    x = torch.randn(2, 64, device="cuda")
    m = stagehand.layer(model, dtype=torch.float32, inference_mode=inference_mode, telemetry=False)
    rt = m._stagehand_layer_runtime
    try:
        with torch.no_grad():
            want = ref(x)
            outs = [m(x) for _ in range(5)]
        for i, y in enumerate(outs):
            assert torch.allclose(y, want, atol=1e-5), f"step {i}"
        if not inference_mode:
            for step in range(2):
                ref.zero_grad(set_to_none=True)
                ref(x).sum().backward()
                for p in model.parameters():
                    p.grad = None
                m(x).sum().backward()
                torch.cuda.synchronize()
                for (name, p), q in zip(model.named_parameters(), ref.parameters()):
                    assert p.grad is not None, (step, name)
                    assert torch.allclose(p.grad.to(q.grad.device), q.grad, atol=1e-5), (step, name)
    finally:
        rt.shutdown()


def test_pinned_pieces_go_straight_to_the_device_after_their_save_back():
    """Pinned host pieces (the outputs of a save-back copy) are copied straight to the device after
    the save-back's event, mixed with pageable pieces that go through slabs, across several slab
    chunks; every byte lands where its piece says."""
    from stagehand_amd.pool import PinnedPool
    from stagehand_amd.transfer import AsyncTransferEngine, BlockSource

    pool = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng = AsyncTransferEngine(pool)
    g = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randint(0, 256, (3 << 19,), dtype=torch.uint8, device="cuda", generator=g)   # 1.5 MiB
    b = torch.randint(0, 256, (5000,), dtype=torch.uint8, device="cuda", generator=g)
    (ha, hb), ev = eng.d2h_async([a, b])
    assert ha.is_pinned() and hb.is_pinned()
    pageable = torch.randint(0, 256, ((5 << 19) + 7,), dtype=torch.uint8)                 # 2.5 MiB + 7
    assert not pageable.is_pinned()
    layout = [(0, ha), (ha.numel(), pageable), (ha.numel() + pageable.numel(), hb)]
    total = sum(t.numel() for _o, t in layout)
    dst = torch.zeros(total, dtype=torch.uint8, device="cuda")
    h = eng.submit_block_load("mixed", BlockSource(layout, total), dst, wait_event=ev)
    eng.wait(h)
    want = torch.cat([a.cpu(), pageable, b.cpu()])
    assert torch.equal(dst.cpu(), want)
    eng.shutdown()
    pool.shutdown()
    # all pinned: no slab is used at all
    pool2 = PinnedPool(total_mb=4, slab_mb=1, alignment=512)
    eng2 = AsyncTransferEngine(pool2)
    dst2 = torch.zeros(ha.numel() + hb.numel(), dtype=torch.uint8, device="cuda")
    h = eng2.submit_block_load("pinned", BlockSource([(0, ha), (ha.numel(), hb)], dst2.numel()), dst2,
                               pinned_pieces=True)
    eng2.wait(h)
    assert torch.equal(dst2.cpu(), torch.cat([a.cpu(), b.cpu()]))
    assert pool2.stats()["peak_in_use"] == 0
    eng2.shutdown()
    pool2.shutdown()


def _sleep_cycles_for(ms: float) -> int:
    """Cycles of torch.cuda._sleep (a bounded spin kernel) that keep the current stream busy for
    about ``ms`` milliseconds on this device."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    probe = 1_000_000
    torch.cuda._sleep(probe)
    start.record()
    torch.cuda._sleep(probe)
    end.record()
    end.synchronize()
    return int(min(probe / max(start.elapsed_time(end), 1e-3) * ms, 4_000_000_000))


def test_save_back_fence_is_the_blocks_last_use_unless_a_parameter_changed():
    """Inside a step, a module-backed block's save-back waits for the block's last hook and the
    step's start, not for the compute queued after them; a parameter changed in place since the
    step began makes it wait for everything queued, so the host copy carries the change (the
    reference copies synchronously at eviction, scheduler.py:1216-1226)."""
    import time

    model = init_(TinyStack(n=3, hidden=64, mlp=2), seed=11).to(torch.bfloat16)
    rt = stagehand.StagehandRuntime(model, _config(prefetch_window_blocks=1), block_pattern=r"^blocks\.\d+$",
                                    dtype=torch.bfloat16, inference_mode=False)
    sched = rt.scheduler
    x = torch.randn(4, 64).to(torch.bfloat16).cuda()
    # a first step evicts blocks 0 and 1 once, so their pinned host buffers exist (allocating
    # pinned memory may wait for the device)
    rt.begin_step(0)
    with torch.no_grad(), rt.managed_forward():
        model(x)
    sched._evict_block("blocks.0", save_back=True)
    sched._evict_block("blocks.1", save_back=True)
    rt.end_step()
    rt.begin_step(1)
    with torch.no_grad(), rt.managed_forward():
        model(x)
    torch.cuda.synchronize()
    names = [n for n, _ in model.blocks[1].named_parameters()]
    want1 = {n: p.detach().cpu().clone() for n, p in model.blocks[1].named_parameters()}
    spin = _sleep_cycles_for(400.0)

    # block 1, unchanged: its save-back completes while the compute stream is still spinning
    torch.cuda._sleep(spin)
    t0 = time.perf_counter()
    sched._evict_block("blocks.1", save_back=True, wait=False)
    t_call = time.perf_counter() - t0
    fence = sched._d2h_fences["blocks.1"]
    while not fence.query() and time.perf_counter() - t0 < 5.0:
        time.sleep(0.001)
    took = time.perf_counter() - t0
    assert took < 0.2, f"the save-back completed after {took * 1e3:.0f} ms (the call took {t_call * 1e3:.0f} ms)"
    for n, p in model.blocks[1].named_parameters():
        assert p.device.type == "cpu" and torch.equal(_bits(p), _bits(want1[n])), n
    torch.cuda.synchronize()

    # block 0, changed in place after its last hook, behind a spin: the copy sees the change
    p0 = dict(model.blocks[0].named_parameters())[names[0]]
    want0 = (p0.detach().float() + 1.0).to(torch.bfloat16).cpu()
    torch.cuda._sleep(spin)
    with torch.no_grad():
        p0.add_(1.0)
    sched._evict_block("blocks.0", save_back=True)
    got = dict(model.blocks[0].named_parameters())[names[0]]
    assert got.device.type == "cpu" and torch.equal(_bits(got), _bits(want0))
    rt.end_step()
    rt.shutdown()


def test_save_back_of_a_block_evicted_while_its_load_is_in_flight():
    """A block evicted right after its load was submitted, never used, is copied back with the
    loaded values: its save-back waits for everything queued, which the eviction ordered after the
    load, and not only for the step's start. The load reads the block's pinned host buffer, which
    the save-back then writes, so a save-back that ran first would put the device's stale bytes
    back into it."""
    model = init_(TinyStack(n=2, hidden=2048, mlp=4), seed=12).to(torch.bfloat16)
    cfg = _config(prefetch_window_blocks=1, pinned_pool_mb=512, pinned_slab_mb=64)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=False)
    sched = rt.scheduler
    x = torch.randn(4, 2048).to(torch.bfloat16).cuda()
    rt.begin_step(0)
    with torch.no_grad(), rt.managed_forward():
        model(x)
    for b in ("blocks.0", "blocks.1"):
        sched._evict_block(b, save_back=True)
    rt.end_step()
    # the host values (views of the block's pinned buffer) change between steps: the device
    # buffer the next load reuses still holds the old ones
    with torch.no_grad():
        for p in model.blocks[0].parameters():
            p.add_(1.0)
    want = {n: p.detach().clone() for n, p in model.blocks[0].named_parameters()}
    rt.begin_step(1)
    torch.cuda._sleep(_sleep_cycles_for(300.0))
    for _ in range(3):
        sched._load_block_to_gpu("blocks.0")
        sched._evict_block("blocks.0", save_back=True)
    for n, p in model.blocks[0].named_parameters():
        assert p.device.type == "cpu" and torch.equal(_bits(p), _bits(want[n])), n
    rt.end_step()
    rt.shutdown()


def test_changed_chunk_save_back_round_trip():
    """Save-backs of the chunks a block changed on the device: the first save-back of a block copies
    it whole into its pinned home buffer; a load from that buffer takes chunk digests; the next
    save-back copies exactly the chunks written since (an in-place change at the first and at the
    last parameter), and one with no change copies nothing. The host values always equal what the
    device held, as after the reference's full copy-back (scheduler.py:1216-1226); a change made to
    the host values between steps travels to the device and is kept."""
    chunk = 4096
    model = init_(TinyStack(n=2, hidden=256, mlp=2), seed=21).to(torch.bfloat16)
    cfg = _config(prefetch_window_blocks=1, save_back_chunk_bytes=chunk)
    rt = stagehand.StagehandRuntime(model, cfg, block_pattern=r"^blocks\.\d+$", dtype=torch.bfloat16,
                                    inference_mode=False)
    sched, eng = rt.scheduler, rt.engine
    block = model.blocks[0]
    x = torch.randn(4, 256).to(torch.bfloat16).cuda()

    def sent(fn):
        torch.cuda.synchronize()
        before = eng.bytes_d2h
        fn()
        sched._sync_d2h_fences()
        eng.reap()
        return eng.bytes_d2h - before

    rt.begin_step(0)
    with torch.no_grad(), rt.managed_forward():
        model(x)
    first = sent(lambda: sched._evict_block("blocks.0", save_back=True))
    rt.end_step()
    size = sum(p.numel() * 2 for p in block.parameters())
    assert first == size  # no home buffer yet: the whole block
    layout = None
    for step in (1, 2):
        rt.begin_step(step)
        sched._load_block_to_gpu("blocks.0")
        sched._await_pending_load("blocks.0")  # the current stream waits for the load on the device
        assert "blocks.0" in sched._load_digests
        layout = sched._residency.get_entry("blocks.0").param_layout
        params = list(block.parameters())
        with torch.no_grad():
            params[0].view(-1)[0] += 1
            params[-1].view(-1)[-1] += 1
        want = [p.detach().cpu().clone() for p in block.parameters()]
        got = sent(lambda: sched._evict_block("blocks.0", save_back=True))
        _name, _shape, dtype, off_last, numel_last = layout[-1]
        dirty = {0, (off_last + (numel_last - 1) * dtype.itemsize) // chunk}
        assert got == sum(min(chunk, size - c * chunk) for c in dirty), (step, got)
        for p, w in zip(block.parameters(), want):
            assert p.device.type == "cpu" and torch.equal(_bits(p), _bits(w))
        rt.end_step()
    # unchanged on the device: nothing copied back
    rt.begin_step(3)
    sched._load_block_to_gpu("blocks.0")
    want = [p.detach().cpu().clone() for p in block.parameters()]
    assert sent(lambda: sched._evict_block("blocks.0", save_back=True)) == 0
    for p, w in zip(block.parameters(), want):
        assert torch.equal(_bits(p), _bits(w))
    rt.end_step()
    # changed on the host while evicted: the load carries it, the digests describe it
    with torch.no_grad():
        for p in block.parameters():
            p.add_(1.0)
    want = [p.detach().clone() for p in block.parameters()]
    rt.begin_step(4)
    sched._load_block_to_gpu("blocks.0")
    sched._await_pending_load("blocks.0")
    dev = [p.detach().cpu() for p in block.parameters()]
    assert all(torch.equal(_bits(a), _bits(b)) for a, b in zip(dev, want))
    assert sent(lambda: sched._evict_block("blocks.0", save_back=True)) == 0
    for p, w in zip(block.parameters(), want):
        assert torch.equal(_bits(p), _bits(w))
    rt.end_step()
    rt.shutdown()


def test_changed_chunk_save_backs_train_bit_identically_to_full_copy_back():
    """The config-5 shape in small, trained twice with every block evicted after every use: once
    with save-backs of changed chunks (the default) and once copying every byte back, as the
    reference does. Outputs, gradients, the updated LoRA weights and the frozen weights' host values
    are bit-identical, and the changed-chunk run moved fewer bytes back."""
    from bench_workloads import TRAIN_BLOCK_PATTERN, TrainDiT, init_train_dit_

    g = torch.Generator().manual_seed(16)
    x = torch.randn(1, 32, 256, generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn(1, 16, 256, generator=g).to(torch.bfloat16).cuda()
    vec = torch.randn(1, 256, generator=g).to(torch.bfloat16).cuda()
    target = torch.randn(1, 32, 256, generator=g).cuda()
    runs = []
    for changed in (True, False):
        # blocks of more than 1 MB: each one alone crosses the high watermark, so every hook evicts
        # every block outside the prefetch window and both runs evict the same blocks
        model = init_train_dit_(TrainDiT(depth=4, hidden=256, heads=4, mlp_ratio=2.0, rank=8), 15)
        assert sum(p.numel() * 2 for p in model.blocks[0].parameters()) > (1 << 20)
        base_mb = int(torch.cuda.memory_allocated() / 2**20)
        cfg = _config(vram_high_watermark_mb=base_mb + 1, vram_low_watermark_mb=base_mb, prefetch_window_blocks=1,
                      save_back_changed_chunks=changed, save_back_chunk_bytes=4096)
        rt = stagehand.StagehandRuntime(model, cfg, block_pattern=TRAIN_BLOCK_PATTERN, dtype=torch.bfloat16,
                                        inference_mode=False)
        lora = [p for n, p in model.named_parameters() if "lora" in n]
        opt = torch.optim.SGD(lora, lr=0.5, foreach=False)
        outs, grads = [], []
        for step in range(3):
            xi = x.clone().requires_grad_()
            rt.begin_step(step)
            with rt.managed_forward(), rt.managed_backward():
                y = model(xi, ctx, vec)
                torch.nn.functional.mse_loss(y.float(), target).backward()
            rt.end_step()
            outs.append(y.detach().cpu())
            grads.append([p.grad.detach().cpu().clone() for p in lora])
            opt.step()
            opt.zero_grad(set_to_none=True)
        torch.cuda.synchronize()
        for i in range(len(model.blocks)):  # the last resident blocks go back too: every host value
            if rt.residency.get_state(f"blocks.{i}").value == "gpu_ready":
                rt.scheduler._evict_block(f"blocks.{i}", save_back=True)
        weights = {n: p.detach().cpu().clone() for n, p in model.named_parameters()}
        runs.append((outs, grads, weights, rt.engine.bytes_d2h, sum(m.evictions for m in rt.telemetry.history)))
        rt.shutdown()
    (o1, g1, w1, d1, e1), (o2, g2, w2, d2, e2) = runs
    assert e1 == e2 and e1 > 0
    for a, b in zip(o1, o2):
        assert torch.equal(_bits(a), _bits(b))
    for ga, gb in zip(g1, g2):
        for a, b in zip(ga, gb):
            assert torch.equal(_bits(a), _bits(b))
    for n in w1:
        assert torch.equal(_bits(w1[n]), _bits(w2[n])), n
    assert d1 < d2
