"""Block streaming state: GPU slots, the copy stream and its event fences -- the drop-in for the reference's
_StreamState (streaming/state.py:21-323), on the direct path (host flats hold the block's compute bytes; one
host -> GPU copy per block into its slot; no staging conversion or scaled-fp8 swaps), with the SSD tier: blocks
without a host flat are read from a file by the native ring, whose uploader thread makes the copy (the role of
_SsdUploader, streaming/ssd_uploader.py:17-120).

Protocol (streaming/state.py:133-161,239-256,294-299 and the hooks of streaming/load_steps.py:451-522):
  issue_prefetch(s): on the copy stream, wait for computed_events[slot] (the slot's previous reader finished),
      copy block s's host flat into slot s % num_slots, record transferred_events[s], query it (forces submission).
  pre-hook of block s: issue the copy if the chain broke, the host waits for transferred_events[s] (host_fence),
      the compute stream waits for it, the block's parameters are bound to the slot's views.
  post-hook of block s: record computed_events[slot] on the compute stream, issue the copy of block s + num_slots.
SSD-tier block s: issue_prefetch records a fresh slot-free event of its own on the compute stream (the slot's
computed event is re-recorded by later blocks, and a copy waiting on a later recording would wait for compute that
needs the copy) and submits the copy to the ring; the pre-hook first waits (host side) until the uploader has put
the copy on the copy stream, then the compute stream waits for transferred_events[s] as for any block.
Copies run on the library's stream with hipMemcpyAsync; the compute stream is torch's current stream."""
import torch

from .. import _native


class _StreamState:
    """Per-model streaming state, owned by one owner token."""

    def __init__(self, owner, device, streaming_blocks, host_flats, host_views, rest, slot_flats, slot_views,
                 is_double=True, ring=None, disk_index=None):
        self.owner = owner
        self.device = torch.device(device)
        self.streaming_blocks = streaming_blocks
        self.host_flats = host_flats      # per block: one flat (pinned) uint8 buffer = copy source
        self.host_views = host_views      # per block: parameter views into host_flats
        self.rest = rest                  # per block: tensors the parameters are bound to between forwards
        self.slot_flats = slot_flats      # per slot: one flat GPU uint8 buffer
        self.slot_views = slot_views      # per slot: parameter views into slot_flats
        self.is_double = is_double
        self.num_stream = len(streaming_blocks)
        self.num_slots = len(slot_flats)
        self.handles = []
        self.profiler = None
        self.prefetch_stream = _native.Stream()
        self.transferred_events = [_native.Event() for _ in range(self.num_stream)]
        self.computed_events = [_native.Event() for _ in range(self.num_slots)]
        # the slots were allocated on the compute stream: the first copy into each waits for the work queued so far
        compute = self.compute_stream()
        for ev in self.computed_events:
            ev.record(compute)
        self.issued = [False] * self.num_stream
        # end of the previous forward on the compute stream: the next forward is enqueued only once it has run
        self.forward_done = _native.Event()
        self.next_issued = set()          # the next forward's blocks already copied (wrap_prefetch)
        self.forward_pending = False
        # The pre-hook's host waits for its block's copy before enqueuing the block (besides the compute stream's
        # wait): measured on MI355X with 40 Wan blocks, the copies then run back to back at the link's 57 GB/s and
        # the step takes 138.9 ms; with the host enqueueing a whole forward ahead, a fifth of the copies ran at
        # 51 GB/s or slower (145-146 ms).
        self.host_fence = True
        self.slot_ptrs = {v.data_ptr() for views in slot_views for v in views}
        self.copies = 0
        # SSD tier: stream index -> position in the ring's block order
        self.ring = ring
        self.disk_index = dict(disk_index or {})
        self.free_events = {s: _native.Event() for s in self.disk_index}
        self.tickets = {}
        self.ssd_submitted = 0

    def compute_stream(self):
        return _native.stream_of(self.device)

    def slot_of(self, s_idx):
        return s_idx % self.num_slots

    def materialize(self, s_idx, slot_idx, stream, next_forward=False):
        """Copy block s_idx's host flat into slot slot_idx on ``stream`` (streaming/state.py:133-149)."""
        prof = self.profiler
        src = self.host_flats[s_idx]
        dst = self.slot_flats[slot_idx]
        n = min(src.numel(), dst.numel())
        if prof is not None:
            prof.record(s_idx, "dma0", stream, next_forward)
        _native.call("wf_h2d_async", dst.data_ptr(), src.data_ptr(), n, stream)
        self.copies += 1
        if prof is not None:
            prof.record(s_idx, "dma1", stream, next_forward)
            prof.record(s_idx, "ready", stream, next_forward)

    def issue_prefetch(self, s_idx):
        """Async copy of block s_idx into its slot, after that slot's last reader finished."""
        if self.profiler is not None:
            self.profiler.mark(s_idx, "cpu_issue")
        slot_idx = self.slot_of(s_idx)
        stream = self.prefetch_stream.handle
        if s_idx in self.disk_index:
            free = self.free_events[s_idx]
            free.record(self.compute_stream())
            self.tickets[s_idx] = self.ring.submit(self.disk_index[s_idx], self.slot_flats[slot_idx], free,
                                                   self.transferred_events[s_idx], stream)
            self.ssd_submitted += 1
            self.copies += 1
            self.issued[s_idx] = True
            return
        _native.stream_wait(stream, self.computed_events[slot_idx])
        self.materialize(s_idx, slot_idx, stream)
        self.transferred_events[s_idx].record(stream)
        self.transferred_events[s_idx].query()        # forces submission without blocking the CPU
        self.issued[s_idx] = True

    def wrap_prefetch(self, slot_idx):
        """At the post-hook of the last block of this forward in slot slot_idx: copy the next forward's block
        slot_idx (the first block that slot serves) into it, so that the next forward starts with its first blocks
        on the GPU instead of waiting for their copies. The captured weights are the same for every forward. Blocks
        of the SSD tier are left to the next forward (the ring serves its blocks in one cycle per forward)."""
        k = slot_idx
        if k >= self.num_stream or k in self.disk_index or self.host_flats[k] is None:
            return
        stream = self.prefetch_stream.handle
        _native.stream_wait(stream, self.computed_events[slot_idx])
        self.materialize(k, slot_idx, stream, next_forward=True)
        self.transferred_events[k].record(stream)
        self.transferred_events[k].query()
        self.next_issued.add(k)

    def wait_transfer(self, s_idx):
        """Host side of the pre-hook for an SSD-tier block: its copy is on the copy stream (the event recorded)."""
        if s_idx in self.disk_index:
            self.ring.wait(self.tickets.pop(s_idx))

    def begin_forward(self):
        """Start of a forward. The host waits until the previous forward has run on the GPU before enqueuing this
        one: measured on MI355X with 40 Wan blocks, a host left to queue forward after forward runs the steps at
        165-171 ms (queued several forwards deep, many block copies ran at 28-40 GB/s), one forward at a time at
        146-148 ms, and with the pre-hooks' host fence as well at 138.8 ms (every copy at 57 GB/s)."""
        if self.forward_pending:
            self.forward_done.synchronize()
            self.forward_pending = False
        self.issued = [s in self.next_issued for s in range(self.num_stream)]
        self.next_issued = set()
        self.ssd_submitted = 0

    def end_forward(self):
        """After a forward: mark its end on the compute stream; when it stopped part way through the SSD tier, let the
        submitted copies finish and restart the ring's cycle at block 0 (DiskRing.restart_if_needed,
        core/tiers/sources.py:318-335)."""
        self.forward_done.record(self.compute_stream())
        self.forward_pending = True
        if self.ring is None:
            return
        pending = list(self.tickets.values())
        self.tickets.clear()
        for t in pending:
            try:
                self.ring.wait(t)
            except _native.NativeError:
                pass
        if pending or self.ssd_submitted % max(1, len(self.disk_index)) != 0:
            self.prefetch_stream.synchronize()
            self.ring.resync()

    def prefetch_first_slots(self):
        """Called when block 0 runs: the first num_slots copies."""
        if self.is_double:
            for s_idx in range(min(self.num_slots, self.num_stream)):
                if not self.issued[s_idx]:
                    self.issue_prefetch(s_idx)

    def restore_rest_binding(self):
        """Rebind every parameter that still points at a GPU slot to its rest tensor (its host view, or for an
        SSD-tier block the tensor it had before streaming)."""
        for blk, rest in zip(self.streaming_blocks, self.rest):
            for p, r in zip(blk.parameters(), rest):
                if p.data.data_ptr() in self.slot_ptrs:
                    p.data = r

    def profile_summary(self):
        return None if self.profiler is None else self.profiler.summary()

    def close(self):
        """Wait for the copies, remove the hooks, drop the events and the stream."""
        if self.ring is not None:
            for t in list(self.tickets.values()):
                try:
                    self.ring.wait(t)
                except _native.NativeError:
                    pass
            self.tickets.clear()
        self.prefetch_stream.synchronize()
        if self.ring is not None:
            self.ring.close()
            self.ring = None
        store = getattr(self, "disk_store", None)
        if store is not None:
            store.delete()
            self.disk_store = None
        for h in self.handles:
            h.remove()
        self.handles = []
        for e in self.transferred_events + self.computed_events + list(self.free_events.values()):
            e.close()
        self.prefetch_stream.close()
        if self.profiler is not None:
            self.profiler.close()
