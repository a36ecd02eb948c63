"""GPU side of the SSD tier: the native ring's uploader (wf_ring_submit / wf_ring_wait) puts each block's file
bytes into its GPU slot, and a streamed forward whose blocks partly come from a GGUF model file through the ring is
bit-identical to the same stack resident on the GPU (the reference's criterion, tests/test_streaming.py:222,
torch.equal) -- over several forwards (the ring's cycle runs on into the next forward), for several ring depths /
reader counts / O_DIRECT settings and SSD layouts, and after a forward that stopped part way (the ring restarts its
cycle); in chunk mode, whose SSD-tier chunks are copied out of the ring's buffers; and with the persistent cache
entry a later load reads instead of writing."""
import numpy as np
import pytest
import torch

from conftest import sub

pytestmark = pytest.mark.gpu


def _stack(n=6, seed=7, qtype=12, mode="fused"):
    syn = sub("streaming.synthetic")
    torch.manual_seed(0)
    m = syn.WanLikeStack(n_blocks=n, dim=512, heads=4, ffn=1024, qtype=qtype, mode=mode)
    m.fill_random(seed)
    return m


def _inputs():
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 256, 512), generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn((1, 64, 512), generator=g).to(torch.bfloat16).cuda()
    return x, ctx


def test_ring_uploads_equal_file_bytes(native, tmp_path):
    src = sub("core.tiers.sources")
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, 6 << 20, dtype=np.uint8)
    p = tmp_path / "blob.bin"
    p.write_bytes(data.tobytes())
    pieces = [[(i * 1_000_003 + 7, 400_000, 0), (i * 1_000_003 + 600_001, 300_000, 409_600)] for i in range(5)]
    source = src.PieceFileSource(str(p), pieces)
    ring = src.DiskRing(source, depth=2, pin=True, threads=2, direct=True)
    stream = native.Stream()
    slots = [torch.zeros(source.block_bytes, dtype=torch.uint8, device="cuda") for _ in range(2)]
    done = [native.Event() for _ in range(2)]
    free = [native.Event() for _ in range(2)]
    try:
        for c in range(3):
            for d in range(5):
                k = (c * 5 + d) % 2
                free[k].record(torch.cuda.current_stream().cuda_stream)
                t = ring.submit(d, slots[k], free[k], done[k], stream.handle)
                ring.wait(t)
                done[k].synchronize()
                got = slots[k].cpu().numpy()
                for o, n, dd in pieces[d]:
                    assert np.array_equal(got[dd:dd + n], data[o:o + n]), (c, d)
        st = ring.stats()
        assert st["reads"] >= 15 and st["bytes"] >= 15 * 700_000
    finally:
        ring.close()
        stream.close()
        for e in done + free:
            e.close()


@pytest.mark.parametrize("ram_blocks,layout,depth,threads,direct", [
    (3, None, 2, 1, True), (3, "tail", 1, 1, False), (1, None, 3, 2, True), (0, None, 2, 2, True)])
def test_streamed_forward_with_ssd_tier_equals_resident(native, tmp_path, ram_blocks, layout, depth, threads, direct):
    dn = sub("streaming.dit_node")
    syn = sub("streaming.synthetic")
    x, ctx = _inputs()
    resident = _stack().cuda()
    with torch.no_grad():
        ref = resident(x, ctx)
    torch.cuda.synchronize()
    model = _stack()
    path = str(tmp_path / "wan6.gguf")
    syn.write_gguf_model(model, path)
    ssd_model = _stack(seed=1)            # other weights in RAM: SSD-tier blocks must come from the file
    ram = set(range(6)) - set(sub("core.tiers.plan").ssd_positions(6, 6 - ram_blocks, layout))
    for i in ram:                          # the RAM tier holds the real weights (captured from the module)
        ssd_model.blocks[i].load_state_dict(model.blocks[i].state_dict())
    sm = dn.apply_streaming(ssd_model, device="cuda", prefetch_slots=2, profile=False, model_file=path,
                            ram_blocks=ram_blocks, ssd_layout=layout, ring_depth=depth, ring_threads=threads,
                            direct_io=direct)
    try:
        assert len(sm.state.disk_index) == 6 - ram_blocks
        for _ in range(3):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
        assert sm.state.ring.stats()["reads"] >= 3 * (6 - ram_blocks)
    finally:
        sm.teardown()


def test_forward_stopped_part_way_restarts_the_ring(native, tmp_path):
    dn = sub("streaming.dit_node")
    syn = sub("streaming.synthetic")
    x, ctx = _inputs()
    resident = _stack().cuda()
    with torch.no_grad():
        ref = resident(x, ctx)
    model = _stack()
    path = str(tmp_path / "wan6.gguf")
    syn.write_gguf_model(model, path)
    sm = dn.apply_streaming(model, device="cuda", prefetch_slots=2, profile=False, model_file=path, ram_blocks=2)
    fail = {"on": True}

    def boom(module, args):
        if fail["on"]:
            raise RuntimeError("stop here")
    h = model.blocks[3].register_forward_pre_hook(boom)
    try:
        with torch.no_grad(), pytest.raises(RuntimeError, match="stop here"):
            sm(x, ctx)
        fail["on"] = False
        for _ in range(2):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    finally:
        h.remove()
        sm.teardown()


def test_file_tensor_size_mismatch_is_rejected(native, tmp_path):
    dn = sub("streaming.dit_node")
    gf = sub("core.tiers.gguf_file")
    syn = sub("streaming.synthetic")
    model = _stack(n=2)
    tensors = syn.gguf_tensors(model)
    tensors = [(n, 0, (q[0],), torch.zeros(q[0] * 4, dtype=torch.uint8)) if n.endswith("q.bias") else (n, t, q, d)
               for n, t, q, d in tensors]           # a bias stored as F32: 4 bytes a value for the parameter's 2
    path = str(tmp_path / "bad.gguf")
    gf.write_gguf(path, tensors, alignment=256)
    with pytest.raises(ValueError, match="bytes"):
        dn.apply_streaming(model, device="cuda", model_file=path, ram_blocks=0)


def test_ssd_tier_from_a_cache_file(native, tmp_path):
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    with torch.no_grad():
        ref = _stack().cuda()(x, ctx)
    torch.cuda.synchronize()
    model = _stack()
    sm = dn.apply_streaming(model, device="cuda", prefetch_slots=2, profile=False, ram_blocks=2,
                            ssd_dir=str(tmp_path / "cache"), ring_depth=2, ring_threads=2)
    path = sm.state.disk_store.path
    try:
        assert len(sm.state.disk_index) == 4 and path.startswith(str(tmp_path))
        for _ in range(3):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    finally:
        sm.teardown()
    import os
    assert not os.path.exists(path)


@pytest.mark.parametrize("ram_blocks,source,slots", [(3, "file", 3), (1, "cache", 2), (0, "file", 4)])
def test_chunk_streaming_with_ssd_tier_equals_resident(native, tmp_path, ram_blocks, source, slots):
    # chunk mode: the SSD-tier blocks' chunks (and, in the calibration forward, their layers) are copied out of the
    # ring's buffers; every forward is bit-identical to the stack resident on the GPU
    dn = sub("streaming.dit_node")
    syn = sub("streaming.synthetic")
    x, ctx = _inputs()
    with torch.no_grad():
        ref = _stack().cuda()(x, ctx)
    torch.cuda.synchronize()
    model = _stack()
    if source == "file":
        path = str(tmp_path / "wan6.gguf")
        syn.write_gguf_model(model, path)
        streamed = _stack(seed=1)          # other weights in RAM: SSD-tier blocks must come from the file
        for i in set(range(6)) - set(sub("core.tiers.plan").ssd_positions(6, 6 - ram_blocks)):
            streamed.blocks[i].load_state_dict(model.blocks[i].state_dict())
        kw = {"model_file": path}
    else:
        streamed, kw = model, {"ssd_dir": str(tmp_path / "cache")}
    print(f"case chunk+ssd ram_blocks={ram_blocks} source={source} slots={slots}", flush=True)
    sm = dn.apply_streaming(streamed, device="cuda", chunk=True, chunk_bytes=300_000, chunk_slots=slots,
                            ram_blocks=ram_blocks, ring_depth=2, ring_threads=2, **kw)
    try:
        assert len(sm.state.disk_index) == 6 - ram_blocks and sm.state.calibrating
        for f in range(4):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f
        assert not sm.state.calibrating and sm.state.n_types >= 2
    finally:
        sm.teardown()


def test_persistent_ssd_cache_reused_by_a_later_load(native, tmp_path, monkeypatch):
    # WEIGHTFERRY_PERSIST_GB: the first load writes the SSD tier's cache entry and keeps it; a later load of the
    # same weights reads it without writing, and both stream bit-identically to the resident stack
    monkeypatch.setenv("WEIGHTFERRY_PERSIST_GB", "1")
    dn = sub("streaming.dit_node")
    cf = sub("core.tiers.cache_files")
    import os
    x, ctx = _inputs()
    with torch.no_grad():
        ref = _stack().cuda()(x, ctx)
    torch.cuda.synchronize()
    paths = []
    for load in range(2):
        sm = dn.apply_streaming(_stack(), device="cuda", ram_blocks=2, ssd_dir=str(tmp_path / "cache"),
                                ring_depth=2, ring_threads=2)
        try:
            if load == 0:
                assert sm.state.disk_store is not None and sm.state.disk_store.keep
                paths.append(sm.state.disk_store.path)

                def no_write(*a, **k):
                    raise AssertionError("written again")
                monkeypatch.setattr(cf.DiskBlockStore, "write_block", no_write)
            else:
                assert sm.state.disk_store is None and sm.state.ring is not None
            for _ in range(2):
                with torch.no_grad():
                    y = sm(x, ctx)
                torch.cuda.synchronize()
                assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), load
        finally:
            sm.teardown()
        assert os.path.exists(paths[0])
