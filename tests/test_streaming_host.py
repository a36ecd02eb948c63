"""Block streaming on the CPU (no GPU): flat layouts (streaming/common.py:99-120 of the reference), and the
prefetch / fence protocol of the hooks (streaming/state.py:239-256, streaming/load_steps.py:451-522) driven through a
recording stand-in for the library's streams, events and copies. The stand-in executes a copy when the stream that
carries it is "run", and a stream runs only past waits whose events have been recorded, so a missing fence shows
up as a block computing with the wrong slot contents."""
import ctypes

import pytest
import torch

from conftest import sub

common = sub("streaming.common")


def test_flat_layout_alignment_and_views():
    specs = [((3, 5), torch.bfloat16), ((7,), torch.uint8), ((2, 2), torch.float32), ((0,), torch.uint8)]
    offsets, total = common._flat_layout(specs)
    assert offsets == [0, 256, 512, 768] and total == 768
    flat = torch.zeros(total, dtype=torch.uint8)
    views = common._views(flat, specs, offsets)
    assert [tuple(v.shape) for v in views] == [(3, 5), (7,), (2, 2), (0,)]
    views[1].fill_(7)
    assert flat[256:263].eq(7).all() and flat[263:512].eq(0).all()
    assert all(o % common._ALIGN == 0 for o in offsets)


class FakeLib:
    """Streams are FIFO queues of ops; events record when the op before them ran. run_all() executes streams in
    round-robin, each as far as its waits allow."""

    def __init__(self):
        self.log = []
        self.queues = {}
        self.recorded = set()
        self.issued = []
        self.next = 1

    def new(self):
        self.next += 1
        return self.next


class FakeNative:
    OK = 0

    def __init__(self):
        self.L = FakeLib()
        outer = self

        class Stream:
            def __init__(self):
                self.handle = outer.L.new()
                outer.L.queues[self.handle] = []

            def synchronize(self):
                outer.run_all()

            def close(self):
                pass

        class Event:
            def __init__(self, timing=False):
                self.handle = outer.L.new()
                self.gen = 0

            def record(self, stream):
                self.gen += 1
                outer.L.queues.setdefault(stream, []).append(("record", self.handle, self.gen))

            def query(self):
                return True

            def synchronize(self):
                outer.run_all()

            def close(self):
                pass

        self.Stream, self.Event = Stream, Event

    def stream_wait(self, stream, event):
        self.L.queues.setdefault(stream, []).append(("wait", event.handle, event.gen))
        self.L.issued.append((stream, "wait", event.handle))

    def call(self, name, *args):
        assert name == "wf_h2d_async"
        dst, src, n, stream = args
        self.L.queues.setdefault(stream, []).append(("copy", dst, src, n))
        self.L.issued.append((stream, "copy", dst))
        return 0

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


class Tagged(torch.nn.Module):
    """A block whose forward checks that its parameters hold its own values (its tag)."""

    def __init__(self, tag, seen):
        super().__init__()
        self.tag = tag
        self.seen = seen
        self.w = torch.nn.Parameter(torch.full((64,), float(tag)), requires_grad=False)
        self.b = torch.nn.Parameter(torch.full((5,), float(tag) * 2), requires_grad=False)

    def forward(self, x):
        self.seen.append((self.tag, float(self.w[0]), float(self.w[-1]), float(self.b[0])))
        return x + self.w.sum()


class Stack(torch.nn.Module):
    def __init__(self, n, seen, skip=()):
        super().__init__()
        self.blocks = torch.nn.ModuleList(Tagged(i + 1, seen) for i in range(n))
        self.skip = set(skip)

    def forward(self, x):
        for i, b in enumerate(self.blocks):
            if i not in self.skip:
                x = b(x)
        return x


@pytest.fixture
def fake(monkeypatch):
    fn = FakeNative()
    state_mod = sub("streaming.state")
    ls_mod = sub("streaming.load_steps")
    monkeypatch.setattr(state_mod, "_native", fn)
    import importlib
    native_real = importlib.import_module("comfyui-weightferry_amd._native")
    monkeypatch.setattr(native_real, "stream_wait", fn.stream_wait)
    monkeypatch.setattr(state_mod._StreamState, "compute_stream", lambda self: 1)
    fn.L.queues[1] = []

    # the compute stream runs its queue every time a block is about to compute (hooks see it via stream_wait)
    orig_pre = ls_mod._install_block_stream_hooks

    def install(dit, state, owner):
        orig_pre(dit, state, owner)
        for blk in state.streaming_blocks:
            blk.register_forward_pre_hook(lambda m, a: fn.run_all())
    monkeypatch.setattr(ls_mod, "_install_block_stream_hooks", install)
    dn = sub("streaming.dit_node")
    monkeypatch.setattr(dn, "_install_block_stream_hooks", install)
    return fn


@pytest.mark.parametrize("slots", [2, 3])
@pytest.mark.parametrize("skip", [(), (3,)])
def test_hook_protocol_binds_the_right_bytes(fake, slots, skip):
    dn = sub("streaming.dit_node")
    seen = []
    model = Stack(7, seen, skip)
    sm = dn.apply_streaming(model, device="cpu", prefetch_slots=slots, pin_memory=False, profile=False)
    for _ in range(2):
        seen.clear()
        sm(torch.zeros(1))
        ran = [i + 1 for i in range(7) if i not in skip]
        assert [s[0] for s in seen] == ran
        for tag, w0, w1, b0 in seen:
            assert (w0, w1, b0) == (tag, tag, 2 * tag), seen
        # after the forward every parameter is bound to its host view again
        for blk, views in zip(model.blocks, sm.state.host_views):
            assert all(p.data.data_ptr() == v.data_ptr() for p, v in zip(blk.parameters(), views))
    assert sm.state.num_slots == slots


def test_self_managed_residents(fake):
    # resident_mode "Self-managed": the resident blocks run on copies of their own, bound for each forward only --
    # what the host application's memory manager then does to the blocks' tensors (a write-back overwriting them)
    # does not reach the forward, and between forwards the parameters hold those tensors again
    dn = sub("streaming.dit_node")
    seen = []
    model = Stack(6, seen)
    own = [[p.data for p in model.blocks[i].parameters()] for i in range(2)]
    sm = dn.apply_streaming(model, device="cpu", resident_blocks=2, prefetch_slots=2, pin_memory=False,
                            profile=False, self_resident=True)
    assert sm.stream_idx == [2, 3, 4, 5]
    for t in own[0] + own[1]:
        t.zero_()                                          # the host application rewrites the blocks' tensors
    for _ in range(2):
        seen.clear()
        sm(torch.zeros(1))
        fake.run_all()
        assert [s[0] for s in seen] == [1, 2, 3, 4, 5, 6]
        for tag, w0, w1, b0 in seen:
            assert (w0, w1, b0) == (tag, tag, 2 * tag), seen
        for i in range(2):
            assert all(p.data_ptr() == t.data_ptr() for p, t in zip(model.blocks[i].parameters(), own[i]))
    sm.teardown(device="cpu")
    assert sm.residents is None
    assert all(p.data_ptr() == t.data_ptr() for p, t in zip(model.blocks[0].parameters(), own[0]))


def test_every_copy_waits_for_the_slots_last_reader(fake):
    dn = sub("streaming.dit_node")
    seen = []
    model = Stack(6, seen)
    sm = dn.apply_streaming(model, device="cpu", prefetch_slots=2, pin_memory=False, profile=False)
    sm(torch.zeros(1))
    fake.run_all()
    copies = [op for op in fake.L.log if op[0] == "copy"]
    # the 6 blocks, then the next forward's blocks 0 and 1 copied by the last block of each slot (wrap_prefetch)
    assert len(copies) == 8
    st = sm.state
    assert st.next_issued == {0, 1}
    assert [op[2] for op in copies[-2:]] == [st.host_flats[0].data_ptr(), st.host_flats[1].data_ptr()]
    slot_of_ptr = {f.data_ptr(): i for i, f in enumerate(st.slot_flats)}
    copy_stream = st.prefetch_stream.handle
    ops = [op for op in fake.L.issued if op[0] == copy_stream]
    for i, op in enumerate(ops):
        if op[1] == "copy":
            slot = slot_of_ptr[op[2]]
            assert i > 0 and ops[i - 1][1] == "wait" and ops[i - 1][2] == st.computed_events[slot].handle
    # the compute stream waits for each block's transfer event before the block runs
    waits = [op[2] for op in fake.L.issued if op[0] == 1 and op[1] == "wait"]
    assert waits == [e.handle for e in st.transferred_events]
    # a second forward starts from the copies made ahead: only blocks 2..5 are copied in it (and again 0, 1 ahead)
    sm(torch.zeros(1))
    fake.run_all()
    assert len([op for op in fake.L.log if op[0] == "copy"]) == 8 + 6


def test_flag_overrides_slot_count(monkeypatch):
    ls = sub("streaming.load_steps")
    monkeypatch.setenv("WEIGHTFERRY_SLOTS", "4")
    assert ls._num_slots(2) == 4
    monkeypatch.delenv("WEIGHTFERRY_SLOTS")
    assert ls._num_slots(1) == 2


def test_layout_mismatch_is_rejected():
    ls = sub("streaming.load_steps")
    a, b = torch.nn.Linear(4, 4), torch.nn.Linear(4, 5)
    with pytest.raises(ValueError):
        ls._check_block_layouts([a, b])


def test_profiler_summary_formulas():
    prof_mod = sub("streaming.profiler")

    class E:
        def __init__(self, t):
            self.t = t

        def elapsed_ms(self, other):
            return other.t - self.t

        def synchronize(self):
            pass

    p = prof_mod._StreamProfiler.__new__(prof_mod._StreamProfiler)
    p.host_bytes, p.is_double, p.no_staging = 1_000_000, True, True
    # two blocks: copies of 2 ms each, the first stalls compute 1 ms, the second not at all
    blocks = {0: {"dma0": E(0), "dma1": E(2), "ready": E(2), "wait0": E(0), "start": E(1), "end": E(4)},
              1: {"dma0": E(2), "dma1": E(4), "ready": E(4), "wait0": E(4), "start": E(4), "end": E(7)}}
    resident = {0: {"r_start": E(8), "r_end": E(9.5)}}
    p.forwards = [prof_mod._Forward(start=E(0), end=E(10), blocks=blocks, resident=resident)]
    summ = p.summary()
    s = summ["per_forward"][0]
    assert s["dma_ms"] == 4 and s["stall_ms"] == 1 and s["streamed_compute_ms"] == 6
    assert s["overlap_ratio"] == 0.75                      # 1 - stall / transfer
    assert s["dma_gbps"] == round(1e6 * 2 / (4 / 1000) / 1e9, 2)
    assert s["resident_compute_ms"] == 1.5 and s["compute_idle_ms"] == 10 - 6 - 1.5
    tl = summ["timeline_one_forward"]
    assert tl["streamed"]["1"]["start"] == 4 and tl["resident"]["0"]["r_end"] == 9.5 and tl["forward_ms"] == 10
    # a stall longer than the copy clamps to 0 hidden; no copy at all gives no ratio and no rate
    blocks[0]["start"] = E(6)
    assert p.summary()["per_forward"][0]["overlap_ratio"] == 0.0
    p.forwards = [prof_mod._Forward(start=E(0), end=E(1), blocks={0: {"start": E(0), "end": E(1)}})]
    s = p.summary()["per_forward"][0]
    assert s["overlap_ratio"] is None and s["dma_gbps"] is None


def test_pinned_host_falls_back_without_gpu():
    pinned = sub("core.tiers.pinned")
    h = pinned.PinnedHost(1000, align=64)
    assert h.tensor.numel() == 1000 and h.tensor.data_ptr() % 64 == 0
    h.tensor.fill_(3)
    h.release()
    assert h.tensor is None
