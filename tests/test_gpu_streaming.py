"""GPU block streaming through the library's pinned buffers, copies and events.

* A streamed forward of a small GGUF DiT stack is bit-identical to the same stack resident on the GPU (the
  reference's own criterion, tests/test_streaming.py:222, torch.equal), with 2 and 3 slots, twice in a row (the
  second forward starting from the first blocks the first one's tail copied ahead), and with a block skipped (the
  prefetch chain repaired in the pre-hook).
* After a copy, a slot holds exactly its block's host bytes.
* The profiler's summary is consistent (overlap in [0, 1], a positive copy rate).
* PinnedHost allocates page-locked memory of the exact size.
"""
import pytest
import torch

from conftest import sub

pytestmark = pytest.mark.gpu


def _small_stack(n=6, mode="fused", qtype=12, seed=7):
    syn = sub("streaming.synthetic")
    torch.manual_seed(0)
    m = syn.WanLikeStack(n_blocks=n, dim=512, heads=4, ffn=1024, qtype=qtype, mode=mode)
    m.fill_random(seed)
    return m


class Skipping(torch.nn.Module):
    def __init__(self, inner, skip):
        super().__init__()
        self.blocks = inner.blocks
        self.skip = set(skip)

    def forward(self, x, ctx):
        for i, b in enumerate(self.blocks):
            if i not in self.skip:
                x = b(x, ctx)
        return x


def _inputs():
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 256, 512), generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn((1, 64, 512), generator=g).to(torch.bfloat16).cuda()
    return x, ctx


@pytest.mark.parametrize("slots", [2, 3])
@pytest.mark.parametrize("mode", ["fused", "dequant"])
def test_streamed_forward_equals_resident(native, slots, mode):
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    resident = _small_stack(mode=mode).cuda()
    with torch.no_grad():
        ref = resident(x, ctx)
    torch.cuda.synchronize()
    streamed = _small_stack(mode=mode)          # same seeds: same weights, on the CPU
    sm = dn.apply_streaming(streamed, device="cuda", prefetch_slots=slots, profile=True)
    try:
        for _ in range(2):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
            for blk in streamed.blocks:       # parameters are back on their host views between forwards
                assert all(p.device.type == "cpu" for p in blk.parameters())
        summ = sm.profile_summary()
        f = summ["per_forward"][-1]
        assert f["streamed_blocks"] == 6 and 0.0 <= f["overlap_ratio"] <= 1.0 and f["dma_gbps"] > 0
        # 6 blocks per forward; the last `slots` blocks of each forward also copy the next forward's first blocks
        assert sm.state.copies == 12 + slots
    finally:
        sm.teardown()


@pytest.mark.parametrize("mode", ["fused", "dequant"])
def test_skipped_block_repairs_the_prefetch_chain(native, mode):
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    resident = Skipping(_small_stack(mode=mode).cuda(), skip=(2,))
    with torch.no_grad():
        ref = resident(x, ctx)
    streamed = Skipping(_small_stack(mode=mode), skip=(2,))
    sm = dn.apply_streaming(streamed, device="cuda", prefetch_slots=2, profile=False)
    try:
        with torch.no_grad():
            y = sm(x, ctx)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    finally:
        sm.teardown()


def test_auto_mode_equals_resident(native):
    # mode "auto": the 256-token linears take the two-step flow, the 64-token cross-attention k / v the fused
    # few-rows kernel; three forwards in a row bit-identical to the resident stack
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    resident = _small_stack(mode="auto").cuda()
    with torch.no_grad():
        ref = resident(x, ctx)
    streamed = _small_stack(mode="auto")
    sm = dn.apply_streaming(streamed, device="cuda", prefetch_slots=2, profile=False)
    try:
        for _ in range(3):
            with torch.no_grad():
                y = sm(x, ctx)
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
        torch.cuda.synchronize()
    finally:
        sm.teardown()


def test_slot_holds_the_blocks_host_bytes(native):
    dn = sub("streaming.dit_node")
    sm = dn.apply_streaming(_small_stack(n=4), device="cuda", prefetch_slots=2, profile=False)
    try:
        st = sm.state
        st.begin_forward()
        for s in range(4):
            st.issue_prefetch(s) if s < 2 else None
        st.prefetch_stream.synchronize()
        for s in range(2):
            assert torch.equal(st.slot_flats[s].cpu(), st.host_flats[s])
        # the next copy into slot 0 waits for computed_events[0]: record it, copy block 2, compare
        st.computed_events[0].record(st.compute_stream())
        st.issue_prefetch(2)
        st.prefetch_stream.synchronize()
        assert torch.equal(st.slot_flats[0].cpu(), st.host_flats[2])
    finally:
        sm.teardown()


def test_pinned_host_is_page_locked(native):
    pinned = sub("core.tiers.pinned")
    before = pinned.registered_bytes()["bytes"]
    h = pinned.PinnedHost(10_000_003)
    assert h.registered and h.tensor.numel() == 10_000_003
    assert pinned.registered_bytes()["bytes"] == before + 10_000_003
    d = torch.empty(10_000_003, dtype=torch.uint8, device="cuda")
    h.tensor.copy_(torch.arange(10_000_003, dtype=torch.int64).to(torch.uint8))
    native.call("wf_h2d_async", d.data_ptr(), h.ptr, 10_000_003, native.stream_of(d.device))
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), h.tensor)
    h.release()
    assert pinned.registered_bytes()["bytes"] == before
    # with an alignment the buffer holds nbytes + align; the counter goes up and back down by that same amount
    h = pinned.PinnedHost(1000, align=256)
    assert h.registered and h.tensor.numel() == 1000 and h.ptr % 256 == 0
    assert pinned.registered_bytes()["bytes"] == before + 1256
    h.release()
    h.release()
    assert pinned.registered_bytes()["bytes"] == before


def test_gguf_linear_fused_matches_dequant_flow(native):
    fg = sub("enhancers.fused_gguf")
    syn = sub("streaming.synthetic")
    for qtype in (12, 13, 14):
        lin = fg.GGUFLinear(512, 768, qtype, bias=True).cuda()
        lin.weight.data.copy_(syn.random_gguf_bytes(768, 512, qtype, seed=qtype).cuda())
        lin.bias.data.normal_(0, 0.1)
        x = torch.randn((3, 100, 512), device="cuda").to(torch.bfloat16)
        y_f = lin(x)
        lin.mode = "dequant"
        y_d = lin(x)
        assert y_f.shape == (3, 100, 768)
        err = (y_f.float() - y_d.float()).abs().max() / y_d.float().abs().max()
        assert err <= 1e-2
        # not the fused kernel's case: float32 activations go through the two-step flow
        assert fg.fused_linear(x.float(), lin.weight, qtype, (768, 512)) is None


@pytest.mark.parametrize("slots,chunk_kb", [(2, 300), (4, 300), (2, 160)])
def test_chunk_streamed_forward_equals_resident(native, slots, chunk_kb):
    # chunk (sub-block) streaming: the first forward learns the call order (copies on the compute stream), the
    # next two stream chunk units through `slots` rotating slots; every forward bit-identical to the resident stack
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    resident = _small_stack(mode="auto").cuda()
    with torch.no_grad():
        ref = resident(x, ctx)
    streamed = _small_stack(mode="auto")
    cache = {}
    sm = dn.apply_streaming(streamed, device="cuda", chunk=True, chunk_bytes=chunk_kb * 1024, chunk_slots=slots,
                            order_cache=cache)
    try:
        for _ in range(3):
            with torch.no_grad():
                y = sm(x, ctx)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
            for blk in streamed.blocks:
                assert all(p.device.type == "cpu" for p in blk.parameters())
        st = sm.state
        assert cache["order"] == ["q", "k", "v", "o", "cq", "ck", "cv", "co", "up", "down"]
        assert st.n_types >= 3 and len(st.chunk_slots) == slots and st.spare_uses == 0
        # registration order = call order: one copy per unit
        assert all(len(plan[0]) == 1 for plan in st.type_plan)
    finally:
        sm.teardown()


def test_chunk_streaming_skipped_block_and_learned_order_reused(native):
    dn = sub("streaming.dit_node")
    x, ctx = _inputs()
    resident = Skipping(_small_stack(mode="auto").cuda(), skip=(2,))
    with torch.no_grad():
        ref = resident(x, ctx)
    cache = {}
    for load in range(2):
        streamed = Skipping(_small_stack(mode="auto"), skip=(2,))
        sm = dn.apply_streaming(streamed, device="cuda", chunk=True, chunk_bytes=300 * 1024, chunk_slots=2,
                                order_cache=cache)
        try:
            # the second load starts chunked: the order the first one learned is reused
            assert sm.state.calibrating == (load == 0)
            for _ in range(2):
                with torch.no_grad():
                    y = sm(x, ctx)
                torch.cuda.synchronize()
                assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
        finally:
            sm.teardown()
