"""Chunk (sub-block) streaming on the CPU (no GPU), driven through the recording stand-in for the library's streams,
events and copies of test_streaming_host (a copy runs when its stream runs; a stream runs only past waits whose
events have been recorded, so a missing fence shows up as a layer computing with the wrong bytes). The protocol is
the reference's streaming/chunk_state.py:124-392: the first forward learns the call order, later forwards copy
chunk units into rotating slots behind slot-free events; layers out of order go through a spare."""
import pytest
import torch

from conftest import sub
from test_streaming_host import FakeNative


class Leaf(torch.nn.Module):
    """A layer whose forward records the first and last value of its weight (its tag when the bytes are right)."""

    def __init__(self, tag, n, seen):
        super().__init__()
        self.tag, self.seen = tag, seen
        self.w = torch.nn.Parameter(torch.full((n,), float(tag)), requires_grad=False)

    def forward(self, x):
        self.seen.append((self.tag, float(self.w[0]), float(self.w[-1])))
        return x + 1


class Blk(torch.nn.Module):
    """Four layers registered a, b, c, d and called in ``order`` (the Cosmos blocks' registration and call orders
    differ too)."""

    def __init__(self, i, seen, order, n=64):
        super().__init__()
        self.a, self.b = Leaf(10 * (i + 1) + 1, n, seen), Leaf(10 * (i + 1) + 2, n, seen)
        self.c, self.d = Leaf(10 * (i + 1) + 3, n, seen), Leaf(10 * (i + 1) + 4, n, seen)
        self.order = order

    def forward(self, x):
        for name in self.order:
            x = getattr(self, name)(x)
        return x


class Model(torch.nn.Module):
    def __init__(self, n, seen, order="cadb", odd=None, outside=False, skip=()):
        super().__init__()
        self.blocks = torch.nn.ModuleList(Blk(i, seen, odd[1] if odd and i == odd[0] else order) for i in range(n))
        self.outside, self.skip = outside, set(skip)

    def forward(self, x):
        if self.outside:
            x = self.blocks[0].c(x)          # a layer of block 0 called before any block runs
        for i, b in enumerate(self.blocks):
            if i not in self.skip:
                x = b(x)
        return x


@pytest.fixture
def fake(monkeypatch):
    fn = FakeNative()
    state_mod = sub("streaming.state")
    chunk_mod = sub("streaming.chunk_state")
    monkeypatch.setattr(state_mod, "_native", fn)
    monkeypatch.setattr(chunk_mod, "_native", fn)
    monkeypatch.setattr(state_mod._StreamState, "compute_stream", lambda self: 1)
    fn.L.queues[1] = []
    ls_mod = sub("streaming.load_steps")
    dn = sub("streaming.dit_node")
    orig = ls_mod._install_chunk_hooks

    def install(dit, state, owner):
        orig(dit, state, owner)
        # the compute stream runs its queue whenever a layer is about to compute
        for mods in state.leaf_modules:
            for m in mods.values():
                m.register_forward_pre_hook(lambda mod, a: fn.run_all())
    monkeypatch.setattr(dn, "_install_chunk_hooks", install)
    return fn


def _check(seen, expect_tags):
    assert [s[0] for s in seen] == expect_tags
    for tag, w0, w1 in seen:
        assert (w0, w1) == (tag, tag), seen


def _tags(n, order, skip=(), outside=False, odd=None):
    idx = {"a": 1, "b": 2, "c": 3, "d": 4}
    out = [13] if outside else []
    for i in range(n):
        if i in skip:
            continue
        o = odd[1] if odd and i == odd[0] else order
        out += [10 * (i + 1) + idx[ch] for ch in o]
    return out


@pytest.mark.parametrize("slots", [2, 3])
def test_learns_call_order_and_binds_the_right_bytes(fake, slots):
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(5, seen)
    cache = {}
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=slots,
                            order_cache=cache)
    st = sm.state
    assert st.calibrating
    for fwd in range(3):
        seen.clear()
        sm(torch.zeros(1))
        fake.run_all()
        _check(seen, _tags(5, "cadb"))
        # after the forward every parameter is bound to its host view again
        for blk, views in zip(model.blocks, st.host_views):
            assert all(p.data.data_ptr() == v.data_ptr() for p, v in zip(blk.parameters(), views))
        if fwd == 0:
            assert not st.calibrating
            assert st.order == ["c", "a", "d", "b"] and cache["order"] == st.order
            assert st.types == [["c", "a"], ["d", "b"]]
            assert len(st.chunk_slots) == slots and len(st.spares) == 1
    assert st.spare_uses == 0
    # parameters a..d are indices 0..3: unit [c, a] is two runs ({0}, {2}), so two copies per unit
    assert [len(plan[0]) for plan in st.type_plan] == [2, 2]


def test_every_copy_waits_for_its_slots_previous_unit(fake):
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(4, seen, order="abcd")
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2)
    sm(torch.zeros(1))                        # calibration
    fake.run_all()
    st = sm.state
    # registration order = call order: each unit is one run, one copy
    assert [len(plan[0]) for plan in st.type_plan] == [1, 1]
    fake.L.issued.clear()
    seen.clear()
    sm(torch.zeros(1))
    fake.run_all()
    _check(seen, _tags(4, "abcd"))
    copy_stream = st.prefetch_stream.handle
    ops = [op for op in fake.L.issued if op[0] == copy_stream]
    slot_of = {b.data_ptr(): k for k, b in enumerate(st.chunk_slots)}
    copies = [i for i, op in enumerate(ops) if op[1] == "copy"]
    assert len(copies) == 4 * 2               # 4 blocks x 2 units, one run each
    for i in copies:
        k = slot_of[ops[i][2]]
        assert ops[i - 1][1] == "wait" and ops[i - 1][2] == st.slot_free_events[k].handle
    # the compute stream waits for each unit's copy before its first layer
    waits = [op[2] for op in fake.L.issued if op[0] == 1 and op[1] == "wait"]
    assert waits == [e.handle for e in st.unit_events]


def test_out_of_order_layers_use_a_spare(fake):
    dn = sub("streaming.dit_node")
    seen = []
    # one layer per unit, two slots: block 2 calls d first, while the rotating slots still hold its c and a units
    model = Model(5, seen, order="cadb", odd=(2, "dcab"))
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=256, chunk_slots=2)
    for _ in range(3):
        seen.clear()
        sm(torch.zeros(1))
        fake.run_all()
        _check(seen, _tags(5, "cadb", odd=(2, "dcab")))
    assert sm.state.types == [["c"], ["a"], ["d"], ["b"]]
    assert sm.state.spare_uses == 2             # once in each chunked forward


def test_skipped_block_and_outside_layer(fake):
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(6, seen, outside=True, skip=(3,))
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2)
    for _ in range(3):
        seen.clear()
        sm(torch.zeros(1))
        fake.run_all()
        _check(seen, _tags(6, "cadb", skip=(3,), outside=True))


def test_order_cache_skips_calibration(fake, monkeypatch):
    dn = sub("streaming.dit_node")
    seen = []
    cache = {"order": ["c", "a", "d", "b"]}
    sm = dn.apply_streaming(Model(3, seen), device="cpu", pin_memory=False, chunk=True, chunk_bytes=512,
                            chunk_slots=2, order_cache=cache)
    assert not sm.state.calibrating and sm.state.types == [["c", "a"], ["d", "b"]]
    sm(torch.zeros(1))
    fake.run_all()
    _check(seen, _tags(3, "cadb"))
    # a stale order (unknown layer names) or the recalibrate flag: learned again
    sm2 = dn.apply_streaming(Model(3, []), device="cpu", pin_memory=False, chunk=True, chunk_bytes=512,
                             chunk_slots=2, order_cache={"order": ["x"]})
    assert sm2.state.calibrating
    monkeypatch.setenv("WEIGHTFERRY_CHUNK_RECALIBRATE", "1")
    sm3 = dn.apply_streaming(Model(3, []), device="cpu", pin_memory=False, chunk=True, chunk_bytes=512,
                             chunk_slots=2, order_cache=dict(cache))
    assert sm3.state.calibrating


def test_stream_waits_alone_are_refused(fake, monkeypatch):
    # the host-side fences are part of the design: the setting that turned them off is refused, not obeyed
    dn = sub("streaming.dit_node")
    monkeypatch.setenv("WEIGHTFERRY_CHUNK_HOST_FENCE", "0")
    with pytest.raises(ValueError, match="HOST_FENCE"):
        dn.apply_streaming(Model(3, []), device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2)
    monkeypatch.setenv("WEIGHTFERRY_CHUNK_HOST_FENCE", "1")
    sm = dn.apply_streaming(Model(3, []), device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2)
    assert sm.state.host_fence


def test_chunk_types_cut_by_bytes():
    chunk = sub("streaming.chunk_state")
    specs = [((64,), torch.float32)] * 3 + [((1000,), torch.float32)]
    offsets = [0, 256, 512, 768]
    runs, where, total = chunk._runs([3, 0, 1], specs, offsets)
    # indices 0, 1 are one run (their padding included), 3 another, placed at the next 256-byte boundary
    assert runs == [(0, 0, 512), (768, 512, 4000)] and where == {0: 0, 1: 256, 3: 512} and total == 4608


def test_chunk_mode_rejects_single_buffer():
    dn = sub("streaming.dit_node")
    with pytest.raises(ValueError):
        dn.apply_streaming(Model(3, []), device="cpu", pin_memory=False, chunk=True, double_buffer=False)


class FakeRing:
    """The native reader ring in host mode (acquire / release) on the CPU: it reads the SSD tier's blocks from the
    source's file into ``depth`` buffers in cyclic order as eagerly as it can -- a buffer is refilled as soon as the
    event its release recorded has run on the stand-in's streams -- so a copy queued out of a buffer after the
    buffer was handed back would read another block's bytes, and a layer would see the wrong tag."""

    fn = None
    made = []

    def __init__(self, source, depth=2, pin=True, threads=1, direct=True, device=None):
        self.source, self.depth, self.n = source, int(depth), source.n_blocks
        self.bufs = [torch.zeros(source.block_bytes, dtype=torch.uint8) for _ in range(self.depth)]
        self.pos = [None] * self.depth            # position each buffer holds
        self.gate = [None] * self.depth           # event a refill waits for
        self.cons = self.reads = self.resyncs = 0
        FakeRing.made.append(self)
        self._refill()

    def _refill(self):
        read_packed = sub("core.tiers.sources").read_packed
        for pos in range(self.cons, self.cons + self.depth):
            b = pos % self.depth
            if self.pos[b] == pos or (self.gate[b] is not None and self.gate[b] not in self.fn.L.recorded):
                continue
            read_packed(self.source, pos % self.n, 0, self.source.block_bytes, self.bufs[b].numpy())
            self.pos[b], self.gate[b] = pos, None
            self.reads += 1

    def acquire(self, d):
        assert d == self.cons % self.n, (d, self.cons)
        b = self.cons % self.depth
        self._refill()
        if self.pos[b] != self.cons:
            self.fn.run_all()                     # the reader waits for the copies out of that buffer
            self._refill()
        assert self.pos[b] == self.cons
        return self.bufs[b], b

    def release(self, slot, stream=None):
        assert slot == self.cons % self.depth and self.pos[slot] == self.cons
        if stream is not None:
            ev = self.fn.Event()
            ev.record(stream)
            self.gate[slot] = (ev.handle, ev.gen)
        self.cons += 1
        self._refill()

    def resync(self):
        self.fn.run_all()
        self.cons, self.resyncs = 0, self.resyncs + 1
        self.pos, self.gate = [None] * self.depth, [None] * self.depth
        self._refill()

    def close(self):
        pass


@pytest.fixture
def ring(fake, monkeypatch):
    FakeRing.fn, FakeRing.made = fake, []
    monkeypatch.setattr(sub("core.tiers.sources"), "DiskRing", FakeRing)
    return FakeRing


@pytest.mark.parametrize("fence", ["1", "0"])
@pytest.mark.parametrize("ram_blocks,depth", [(3, 2), (1, 3), (4, 2)])
def test_ssd_tier_chunks_come_out_of_the_ring(ring, monkeypatch, tmp_path, fence, ram_blocks, depth):
    # 6 streamed blocks, some on the SSD tier (a cache file of their captured bytes): the calibration forward and
    # the chunked ones copy their units out of the ring's buffers; every layer sees its own bytes, with or without
    # the host fences, and the ring serves each SSD-tier block once per forward
    monkeypatch.setattr(sub("streaming.chunk_state")._ChunkState, "host_fence", fence == "1")
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(6, seen)
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2,
                            ram_blocks=ram_blocks, ring_depth=depth, ssd_dir=str(tmp_path))
    st = sm.state
    n_disk = 6 - ram_blocks
    assert len(st.disk_index) == n_disk and all(st.host_flats[s] is None for s in st.disk_index)
    r = ring.made[0]
    for _ in range(4):
        seen.clear()
        sm(torch.zeros(1))
        ring.fn.run_all()
        _check(seen, _tags(6, "cadb"))
        assert r.cons % n_disk == 0 and st._held is None
    assert r.resyncs == 0 and r.cons == 4 * n_disk
    # parameters of SSD-tier blocks go back to their own tensors between forwards
    for s in st.disk_index:
        assert all(p.data.data_ptr() == t.data_ptr() for p, t in zip(model.blocks[s].parameters(), st.rest[s]))
    sm.teardown(device="cpu")


def test_ssd_tier_chunks_with_skipped_block_and_outside_layer(ring, tmp_path):
    # blocks 0, 2, 3 and 5 on the SSD tier: the forward skips block 3 (the ring reads it and hands it straight
    # back) and calls a layer of block 0 before any block (read from the file, not through the ring)
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(6, seen, outside=True, skip=(3,))
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2,
                            ram_blocks=2, ssd_dir=str(tmp_path))
    assert sorted(sm.state.disk_index) == [0, 2, 3, 5]
    for _ in range(3):
        seen.clear()
        sm(torch.zeros(1))
        ring.fn.run_all()
        _check(seen, _tags(6, "cadb", skip=(3,), outside=True))
    assert ring.made[0].resyncs == 0 and ring.made[0].cons == 3 * 4


def test_ssd_tier_forward_stopped_part_way(ring, tmp_path):
    # a forward that fails in block 3: the ring's cycle restarts, and the next forwards are right
    dn = sub("streaming.dit_node")
    seen = []
    model = Model(6, seen)

    def boom(mod, args):
        if getattr(model, "fail", False):
            raise RuntimeError("stop")
    model.blocks[3].register_forward_pre_hook(boom)
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=512, chunk_slots=2,
                            ram_blocks=2, ssd_dir=str(tmp_path))
    sm(torch.zeros(1))                            # calibration
    model.fail = True
    with pytest.raises(RuntimeError):
        sm(torch.zeros(1))
    model.fail = False
    assert ring.made[0].resyncs == 1
    for _ in range(2):
        seen.clear()
        sm(torch.zeros(1))
        ring.fn.run_all()
        _check(seen, _tags(6, "cadb"))


class DeferredFake(FakeNative):
    """The stand-in with layer reads deferred onto the compute stream: a layer's forward enqueues a read of its
    weight tensor, executed when the stream runs, as a kernel would read it -- so the host can run a whole forward
    ahead of the "GPU", which only runs at the end of each forward (the host's forward_done wait)."""

    def run_all(self):
        progress = True
        while progress:
            progress = False
            for s, q in self.L.queues.items():
                while q:
                    op = q[0]
                    if op[0] == "wait" and (op[1], op[2]) not in self.L.recorded and op[2] > 0:
                        break
                    q.pop(0)
                    progress = True
                    if op[0] == "record":
                        self.L.recorded.add((op[1], op[2]))
                    elif op[0] == "copy":
                        ctypes.memmove(op[1], op[2], op[3])
                        self.L.log.append(("copy", op[1], op[2]))
                    elif op[0] == "fn":
                        op[1]()


import ctypes  # noqa: E402


class DLeaf(torch.nn.Module):
    def __init__(self, tag, n, seen, fake):
        super().__init__()
        self.tag, self.seen, self.fake = tag, seen, fake
        self.w = torch.nn.Parameter(torch.full((n,), float(tag)), requires_grad=False)

    def forward(self, x):
        w, tag = self.w.data, self.tag
        self.fake.L.queues[1].append(("fn", lambda: self.seen.append((tag, float(w[0]), float(w[-1])))))
        return x


class WanLike(torch.nn.Module):
    """Ten layers per block sized like a Wan block's (eight of 14.76 units, up and down 39.8), called in order."""

    def __init__(self, i, seen, fake):
        super().__init__()
        sizes = [1476] * 8 + [3980, 3980]
        self.layers = torch.nn.ModuleList(DLeaf(100 * (i + 1) + k, n, seen, fake) for k, n in enumerate(sizes))

    def forward(self, x):
        for m in self.layers:
            x = m(x)
        return x


@pytest.mark.parametrize("blocks,slots,chunk_kb,ram_blocks,fence", [
    (40, 4, 38, None, "1"), (12, 4, 38, None, "1"), (40, 2, 38, None, "1"), (40, 4, 17, None, "1"),
    (40, 4, 38, None, "0"), (12, 4, 38, 6, "0"), (12, 2, 17, 3, "0"), (40, 4, 38, 20, "0"), (12, 4, 38, 6, "1")])
def test_host_far_ahead_of_the_gpu(monkeypatch, tmp_path, blocks, slots, chunk_kb, ram_blocks, fence):
    # the whole forward is enqueued before anything runs (without the host fences: nothing runs until the forward's
    # end); every layer must still read its own bytes -- with SSD-tier blocks too, whose ring buffers are refilled
    # as soon as the copies queued out of them have run
    monkeypatch.setattr(sub("streaming.chunk_state")._ChunkState, "host_fence", fence == "1")
    fn = DeferredFake()
    FakeRing.fn, FakeRing.made = fn, []
    monkeypatch.setattr(sub("core.tiers.sources"), "DiskRing", FakeRing)
    state_mod = sub("streaming.state")
    chunk_mod = sub("streaming.chunk_state")
    monkeypatch.setattr(state_mod, "_native", fn)
    monkeypatch.setattr(chunk_mod, "_native", fn)
    monkeypatch.setattr(state_mod._StreamState, "compute_stream", lambda self: 1)
    fn.L.queues[1] = []
    dn = sub("streaming.dit_node")
    seen = []

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList(WanLike(i, seen, fn) for i in range(blocks))

        def forward(self, x):
            for b in self.blocks:
                x = b(x)
            return x

    model = M()
    sm = dn.apply_streaming(model, device="cpu", pin_memory=False, chunk=True, chunk_bytes=chunk_kb * 1024,
                            chunk_slots=slots, ram_blocks=ram_blocks, ssd_dir=str(tmp_path))
    assert len(sm.state.disk_index) == (0 if ram_blocks is None else blocks - ram_blocks)
    for f in range(5):
        seen.clear()
        sm(torch.zeros(1))
        fn.run_all()
        bad = [(t, a, b) for t, a, b in seen if (a, b) != (t, t)]
        assert not bad, (f, bad[:4])
        assert len(seen) == blocks * 10
