"""The WeightFerryDiT node on the GPU through a stand-in ModelPatcher (ON_LOAD / ON_DETACH callbacks and the
DIFFUSION_MODEL wrapper, as ComfyUI calls them): every forward is bit-identical to the same stack resident on the GPU
(the reference's criterion, tests/test_streaming.py:222) -- after a load, twice; when ComfyUI skipped ON_LOAD (lazy
capture in the wrapper); with Single Buffer; after a re-load; with tiering Auto putting blocks over the RAM
budget on the SSD tier (read from the GGUF file); and in chunk mode (WEIGHTFERRY_CHUNK=1, block 0 streamed too, the
learned call order reused by a re-load), with tiering Auto as well. A detach gives the weights back on the CPU."""
import pytest
import torch

from conftest import sub

import fake_comfy

pytestmark = pytest.mark.gpu


@pytest.fixture
def comfy():
    fake_comfy.make_comfy_modules()
    yield
    fake_comfy.remove_comfy_modules()


def _stack(n=6, seed=7):
    syn = sub("streaming.synthetic")
    torch.manual_seed(0)
    m = syn.WanLikeStack(n_blocks=n, dim=512, heads=4, ffn=1024, qtype=12)
    m.fill_random(seed)
    return m


def _inputs():
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 256, 512), generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn((1, 64, 512), generator=g).to(torch.bfloat16).cuda()
    return x, ctx


@pytest.fixture
def reference():
    x, ctx = _inputs()
    with torch.no_grad():
        ref = _stack().cuda()(x, ctx)
    torch.cuda.synchronize()
    return x, ctx, ref


def _check(mp, x, ctx, ref, times=2):
    for _ in range(times):
        with torch.no_grad():
            y = mp.apply_model(x, ctx)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("buffer_mode,slots", [("Double Buffer (Async Prefetch, Recommended)", 3),
                                               ("Double Buffer (Async Prefetch, Recommended)", 2),
                                               ("Single Buffer (Synchronous)", 3)])
def test_load_forward_detach(native, comfy, reference, buffer_mode, slots):
    x, ctx, ref = reference
    node = sub("streaming.node")
    model = _stack()
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=1,
                                               buffer_mode=buffer_mode, prefetch_slots=slots)[0]
    model.blocks[0].cuda()                      # ComfyUI loads the resident part before ON_LOAD
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    assert len(sm.stream_idx) == 5 and sm.state.num_slots == (slots if "Double" in buffer_mode else 1)
    _check(mp, x, ctx, ref)
    mp.detach()
    assert getattr(model, node._NODE_ATTR) is None
    assert all(p.device.type == "cpu" for b in model.blocks[1:] for p in b.parameters())


def test_self_managed_residents(native, comfy, reference):
    # resident_mode "Self-managed": the two resident blocks run on the node's own GPU copies, bound for each forward
    # only; a write-back into the blocks' own tensors between forwards does not change the output
    x, ctx, ref = reference
    node = sub("streaming.node")
    model = _stack()
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=2,
                                               resident_mode=node.RESIDENT_MODE_SELF, prefetch_slots=2)[0]
    model.blocks[0].cuda()
    model.blocks[1].cuda()
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    assert sm.residents is not None and len(sm.stream_idx) == 4
    _check(mp, x, ctx, ref, times=1)
    for p in model.blocks[1].parameters():
        p.data.zero_()
    _check(mp, x, ctx, ref, times=2)
    mp.detach()
    assert all(p.device.type == "cpu" for b in model.blocks for p in b.parameters())


def test_skipped_on_load_captures_lazily(native, comfy, reference):
    x, ctx, ref = reference
    node = sub("streaming.node")
    model = _stack()
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=2)[0]
    model.blocks[0].cuda()
    model.blocks[1].cuda()
    _check(mp, x, ctx, ref)                     # no load(): the wrapper captures at the first forward
    mp.load()                                   # a re-load tears the capture down and captures again
    _check(mp, x, ctx, ref)
    mp.detach()


def _reference10():
    x, ctx = _inputs()
    with torch.no_grad():
        ref = _stack(n=10).cuda()(x, ctx)
    torch.cuda.synchronize()
    return x, ctx, ref


def test_tiering_auto_reads_blocks_over_the_budget_from_the_file(native, comfy, tmp_path, monkeypatch):
    x, ctx, ref = _reference10()
    node = sub("streaming.node")
    syn = sub("streaming.synthetic")
    model = _stack(n=10)
    path = str(tmp_path / "wan10.gguf")
    syn.write_gguf_model(model, path)
    per_block = sum(p.numel() * p.element_size() for p in model.blocks[1].parameters())
    monkeypatch.setenv("WEIGHTFERRY_MODEL_FILE", path)
    monkeypatch.setenv("WEIGHTFERRY_DISK_PROBE_MB", "16")
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=1,
                                               tiering="Auto (GPU / RAM / SSD)",
                                               ram_budget_gb=6.5 * per_block / 1024 ** 3)[0]
    model.blocks[0].cuda()
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    # 9 streamed blocks; the budget holds the ring (4 buffers) and 2 blocks
    assert len(sm.state.disk_index) == 7 and sm.state.ring.depth == 4
    _check(mp, x, ctx, ref, times=3)
    mp.detach()


def test_tiering_auto_without_a_model_file_uses_a_cache_file(native, comfy, tmp_path, monkeypatch):
    x, ctx, ref = _reference10()
    node = sub("streaming.node")
    model = _stack(n=10)
    per_block = sum(p.numel() * p.element_size() for p in model.blocks[1].parameters())
    monkeypatch.delenv("WEIGHTFERRY_MODEL_FILE", raising=False)
    monkeypatch.setenv("WEIGHTFERRY_CACHE_DIR", str(tmp_path / "cache"))
    monkeypatch.setenv("WEIGHTFERRY_DISK_PROBE_MB", "16")
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=1,
                                               tiering="Auto (GPU / RAM / SSD)",
                                               ram_budget_gb=5.5 * per_block / 1024 ** 3)[0]
    model.blocks[0].cuda()
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    assert len(sm.state.disk_index) == 8 and sm.state.disk_store is not None     # ring of 4 and 1 block in RAM
    _check(mp, x, ctx, ref, times=2)
    mp.detach()


def test_chunk_mode_streams_block0_and_reuses_the_order(native, comfy, reference, monkeypatch):
    x, ctx, ref = reference
    node = sub("streaming.node")
    monkeypatch.setenv("WEIGHTFERRY_CHUNK", "1")
    monkeypatch.setenv("WEIGHTFERRY_CHUNK_MB", "0.3")
    model = _stack()
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=1)[0]
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    assert len(sm.stream_idx) == 6 and sm.state.chunk_mode and sm.state.calibrating
    _check(mp, x, ctx, ref, times=3)
    mp.load()                                   # a re-load: chunked from its first forward
    sm = getattr(model, node._NODE_ATTR)
    assert not sm.state.calibrating and sm.state.n_types >= 3
    _check(mp, x, ctx, ref, times=2)
    mp.detach()
    assert all(p.device.type == "cpu" for b in model.blocks for p in b.parameters())


def test_chunk_mode_with_tiering_auto(native, comfy, tmp_path, monkeypatch):
    # WEIGHTFERRY_CHUNK=1 and tiering Auto: the blocks over the budget go to the SSD tier (a cache file), whose
    # chunks come out of the reader ring; the ring's readers follow the drive probe (kept in the cache folder)
    x, ctx, ref = _reference10()
    node = sub("streaming.node")
    model = _stack(n=10)
    per_block = sum(p.numel() * p.element_size() for p in model.blocks[1].parameters())
    monkeypatch.delenv("WEIGHTFERRY_MODEL_FILE", raising=False)
    monkeypatch.setenv("WEIGHTFERRY_CACHE_DIR", str(tmp_path / "cache"))
    monkeypatch.setenv("WEIGHTFERRY_DISK_PROBE_MB", "16")
    monkeypatch.setenv("WEIGHTFERRY_CHUNK", "1")
    monkeypatch.setenv("WEIGHTFERRY_CHUNK_MB", "0.3")
    mp = node.WeightFerryDiT().apply_streaming(fake_comfy.FakeModelPatcher(model), resident_blocks=1,
                                               tiering="Auto (GPU / RAM / SSD)",
                                               ram_budget_gb=6.5 * per_block / 1024 ** 3)[0]
    mp.load()
    sm = getattr(model, node._NODE_ATTR)
    assert sm.state.chunk_mode and len(sm.state.disk_index) >= 4
    import os
    assert os.path.exists(str(tmp_path / "cache" / "weightferry_disk_probe.json"))
    _check(mp, x, ctx, ref, times=3)
    mp.detach()
    assert all(p.device.type == "cpu" for b in model.blocks for p in b.parameters())
