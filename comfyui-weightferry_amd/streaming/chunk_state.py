"""Chunk (sub-block) streaming: the GPU holds a few chunks of a block's layers instead of whole blocks -- the role
of the reference's _ChunkState (streaming/chunk_state.py:22-519).

A block's layers ("leaves": the modules that own parameters directly) are cut into chunk types along the order in
which the block really calls them, consecutive leaves up to ``chunk_bytes`` per type. That order is learned in the
first forward ("calibration", streaming/chunk_state.py:124-143): each leaf's parameters are copied on the compute
stream into a scratch buffer just before the leaf runs, and the call order of the first streamed block is recorded.
It can be kept with the model (``order_cache``, a dict) so that a later load starts chunked at once
(streaming/chunk_state.py:155-168); WEIGHTFERRY_CHUNK_RECALIBRATE=1 learns it again.

Chunked forwards: unit u = block s x type t (u = s * n_types + t) is copied into rotating slot u % num_slots on the
copy stream after that slot's previous unit finished (its slot-free event, recorded on the compute stream when every
leaf of that unit has run, or when its block ends); the compute stream waits for the unit's copy event before the
first of its leaves runs, and the unit's parameters are bound to the slot's views (streaming/chunk_state.py:259-392).
A unit whose rotating slot is still held when one of its leaves is called (a layer out of the learned order) goes
into a spare buffer; a spare is reused only once its unit has finished, and another is allocated when none is free.
A leaf called before any block of the forward has started (a caching wrapper calling block 0's modulation on its
own) is copied on the compute stream into a buffer of its own and not counted against its unit
(streaming/chunk_state.py:405-432).

Copies: a unit's parameters are grouped into runs of consecutive parameters of the block's flat host layout; each run
is one hipMemcpyAsync of the host bytes (alignment padding included) into the slot, placed so every parameter keeps
its 256-byte alignment. When a block calls its layers in registration order, a unit is one copy.

SSD tier: a block without a host flat is read by the native ring (host mode: acquire / release), in the tier's
order; the ring buffer holding it is the copy source of its units (and of its layers in the calibration forward)
until a unit of the next SSD-tier block needs the ring, and is handed back after the copies queued out of it (on
every stream that copied from it). Blocks a forward skips are read and handed straight back, so the ring stays in
step; a forward that stops before the tier's last block restarts the ring's cycle. A unit is never copied for a
block that has finished: when a block starts, units of earlier blocks that were not copied are dropped for this
forward. A layer of an SSD-tier block called before any block of the forward is read from the file on its own (not
through the ring, which is in the tier's order).

Not supported here (block streaming is used instead): the single-buffer mode, the profiler."""
import time

import torch

from .. import _native
from ..core import env as _env
from ..utils.logging import log_info
from .common import _align_up, _nbytes
from .state import _StreamState


def _runs(js, specs, offsets):
    """Copy plan of the parameters ``js`` (indices into the block's flat layout): runs of consecutive indices, each
    copied as one byte range. Returns (runs [(host_offset, buffer_offset, nbytes)], {j: buffer_offset}, total)."""
    runs, where, base, cur = [], {}, 0, []
    for j in sorted(set(js)) + [None]:
        if cur and (j is None or j != cur[-1] + 1):
            h0 = offsets[cur[0]]
            h1 = offsets[cur[-1]] + _nbytes(*specs[cur[-1]])
            for i in cur:
                where[i] = base + offsets[i] - h0
            runs.append((h0, base, h1 - h0))
            base = _align_up(base + h1 - h0)
            cur = []
        if j is not None:
            cur.append(j)
    return runs, where, base


def _pack(order, size_of, limit):
    """Chunk types: ``order`` cut into consecutive runs of leaves, each run closed before the leaf that would take it
    past ``limit`` bytes (a leaf larger than ``limit`` makes a run of its own)."""
    cuts, filled = [0], 0
    for i, leaf in enumerate(order):
        if i > cuts[-1] and filled + size_of[leaf] > limit:
            cuts.append(i)
            filled = 0
        filled += size_of[leaf]
    cuts.append(len(order))
    return [list(order[a:b]) for a, b in zip(cuts, cuts[1:])]


def _stored_order(order_cache, leaves):
    """The leaf call order an earlier load kept in ``order_cache``, when there is one that names only these blocks'
    leaves and WEIGHTFERRY_CHUNK_RECALIBRATE=1 does not ask to learn it again; else None."""
    if order_cache is None or _env.get("WEIGHTFERRY_CHUNK_RECALIBRATE") == "1":
        return None
    kept = order_cache.get("order") or ()
    if not kept or any(leaf not in leaves for leaf in kept):
        return None
    return list(kept)


class _ChunkState(_StreamState):
    """Per-model chunk streaming state (double-buffered, RAM tier)."""

    # The host waits for the slot-free event before a unit's copy is issued and for the unit's copy event before its
    # first leaf runs, besides the two stream waits. Required: with the stream waits alone, 40 Wan blocks streamed in
    # 3 chunks each gave layers wrong bytes on MI355X (every forward on one machine, none on others), never with one
    # hardware queue (GPU_MAX_HW_QUEUES=1) and never in the CPU model of the queues. The cause is not known. Only that
    # CPU model (tests) clears this flag, to check the stream-wait ordering of the protocol by itself.
    host_fence = True

    def __init__(self, owner, device, streaming_blocks, host_flats, host_views, rest, specs, offsets, chunk_bytes,
                 num_slots, order_cache=None, ring=None, disk_index=None, source=None):
        super().__init__(owner, device, streaming_blocks, host_flats, host_views, rest, [], [], True, ring=ring,
                         disk_index=disk_index)
        self.source = source
        self._held = None                 # [block, host address, ring slot, streams that copied from it]
        self._ring_next = 0               # position in the SSD tier of the next block the ring serves
        self._staging = None              # (pinned buffer, event of its last copy) for layers read outside the ring
        self.chunk_mode = True
        self.specs, self.offsets = specs, offsets
        self.chunk_bytes = int(chunk_bytes)
        self.n_chunk_slots = max(2, int(num_slots))
        names = [n for n, _ in streaming_blocks[0].named_parameters()]
        if not names:
            raise ValueError("chunk streaming needs blocks with parameters")
        self.leaf_params = {}
        for j, n in enumerate(names):
            self.leaf_params.setdefault(n.rpartition(".")[0], []).append(j)
        self.block_params = [list(b.parameters()) for b in streaming_blocks]
        self.leaf_modules = [{leaf: (b.get_submodule(leaf) if leaf else b) for leaf in self.leaf_params}
                             for b in streaming_blocks]
        self.mod_info = {id(m): (s, leaf) for s, mods in enumerate(self.leaf_modules) for leaf, m in mods.items()}
        self.leaf_plan = {leaf: _runs(js, specs, offsets) for leaf, js in self.leaf_params.items()}
        self.leaf_bytes = {leaf: plan[2] for leaf, plan in self.leaf_plan.items()}
        max_leaf = max(self.leaf_bytes.values())
        self.scratch = torch.empty(max_leaf, dtype=torch.uint8, device=self.device)
        self.scratch_views = {leaf: self._views(self.scratch, plan[1]) for leaf, plan in self.leaf_plan.items()}
        self.outside_buf = None
        self.calibrating = True
        self.order = []                   # leaves of the first streamed block in first-call order
        self.types = None                 # chunk types: [[leaf, ...], ...]
        self.type_of_leaf = {}
        self.chunk_slots = []
        self.spares = []                  # [(buffer, free event, per-type views)]
        self.order_cache = order_cache
        self.spare_uses = 0
        self.blocks_started = 0
        self._fwd = None
        self._retired = []                # unit events replaced in this forward (closed once it has run)
        if _env.get("WEIGHTFERRY_CHUNK_HOST_FENCE") == "0":
            raise ValueError("WEIGHTFERRY_CHUNK_HOST_FENCE=0 is not supported: chunk copies ordered by stream waits "
                             "alone gave layers wrong bytes on MI355X, so the host-side fences always stay on")
        kept = _stored_order(order_cache, self.leaf_params)
        if kept is not None:
            self.order = kept
            self.finish_calibration()
            log_info(f"DiT Layer Streaming [chunks]: {len(kept)} leaves in the stored call order; chunked from the "
                     f"first forward.")

    # ---- helpers
    def _views(self, buf, where):
        """{j: typed view} of the parameters placed in ``buf`` at the offsets ``where``."""
        return [(j, buf[o:o + _nbytes(*self.specs[j])].view(self.specs[j][1]).view(self.specs[j][0]))
                for j, o in sorted(where.items())]

    def _bind(self, s, pairs):
        params = self.block_params[s]
        for j, view in pairs:
            params[j].data = view

    def _copy(self, s, runs, dst, stream, src=None):
        if src is None:
            src = self._host_base(s, stream)
        base = dst.data_ptr()
        for host_off, buf_off, n in runs:
            _native.call("wf_h2d_async", base + buf_off, src + host_off, n, stream)
            self.copies += 1

    # ---- the SSD tier's ring
    def _host_base(self, s, stream):
        """Host address of block s's packed bytes for a copy on ``stream``: its pinned flat, or the ring buffer
        holding it (the ring is moved on to it first)."""
        if s not in self.disk_index:
            return self.host_flats[s].data_ptr()
        if self._held is None or self._held[0] != s:
            self._ring_release()
            d, n = self.disk_index[s], len(self.disk_index)
            while self._ring_next != d:   # SSD-tier blocks this forward skipped
                _, slot = self.ring.acquire(self._ring_next)
                self.ring.release(slot)
                self._ring_next = (self._ring_next + 1) % n
            buf, slot = self.ring.acquire(d)
            self._ring_next = (d + 1) % n
            self._held = [s, buf.data_ptr(), slot, set()]
        self._held[3].add(stream)
        return self._held[1]

    def _ring_release(self):
        """Hand the held ring buffer back, refilled only after every copy queued out of it."""
        if self._held is None:
            return
        _, _, slot, streams = self._held
        self._held = None
        streams = sorted(streams)
        last = streams[-1]
        for other in streams[:-1]:
            ev = _native.Event()
            ev.record(other)
            _native.stream_wait(last, ev)
            self._retired.append(ev)
        self.ring.release(slot, last)

    def _staged_copy(self, s, runs, dst, stream):
        """Copy runs of SSD-tier block s into ``dst`` on ``stream`` from the file itself (via the staging buffer),
        leaving the ring where it is."""
        src, runs = self._read_outside(s, runs)
        self._copy(s, runs, dst, stream, src=src)
        ev = _native.Event()
        ev.record(stream)
        if self._staging[1] is not None:
            self._retired.append(self._staging[1])
        self._staging = (self._staging[0], ev)

    def _read_outside(self, s, runs):
        """Runs of an SSD-tier block read from the source file into the pinned staging buffer, back to back (after
        the staging buffer's previous copy); returns (staging address, runs re-based on it)."""
        from ..core.tiers.sources import read_packed
        total = sum(n for _, _, n in runs)
        if self._staging is None or self._staging[0].numel() < total:
            size = max(total, max(self.leaf_bytes.values()))
            buf = torch.empty(size, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
            self._staging = (buf, None)
        buf, ev = self._staging
        if ev is not None:
            ev.synchronize()
        out, pos = [], 0
        for host_off, buf_off, n in runs:
            read_packed(self.source, self.disk_index[s], host_off, n, buf[pos:pos + n].numpy())
            out.append((pos, buf_off, n))
            pos += n
        return buf.data_ptr(), out

    # ---- calibration (the first forward after the capture)
    def _calib_leaf_pre(self, module):
        s, leaf = self.mod_info[id(module)]
        if s == 0 and leaf not in self.order:
            self.order.append(leaf)
        # on the compute stream: ordered after every kernel of the previous leaf that read the scratch buffer
        compute = self.compute_stream()
        if s in self.disk_index and self.blocks_started == 0:
            self._staged_copy(s, self.leaf_plan[leaf][0], self.scratch, compute)
        else:
            self._copy(s, self.leaf_plan[leaf][0], self.scratch, compute)
        self._bind(s, self.scratch_views[leaf])

    def finish_calibration(self):
        """Chunk types from the learned order (leaves never called go last, in registration order), their copy
        plans, the slots and the events; the order is kept in ``order_cache`` for later loads."""
        if self.order and self.order_cache is not None:
            self.order_cache["order"] = list(self.order)
        called = set(self.order)
        types = _pack(list(self.order) + [leaf for leaf in self.leaf_params if leaf not in called], self.leaf_bytes,
                      self.chunk_bytes)
        self.types = types
        self.n_types = len(types)
        self.type_of_leaf = {leaf: t for t, leaves in enumerate(types) for leaf in leaves}
        self.type_plan = [_runs([j for leaf in leaves for j in self.leaf_params[leaf]], self.specs, self.offsets)
                          for leaves in types]
        self.slot_bytes = max(plan[2] for plan in self.type_plan)
        self.chunk_slots = [torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
                            for _ in range(self.n_chunk_slots)]
        self.slot_type_views = [[self._views(buf, plan[1]) for plan in self.type_plan] for buf in self.chunk_slots]
        # the slots come from the compute stream's allocator: a first copy into each waits for the work queued so far
        compute = self.compute_stream()
        self.slot_free_events = [_native.Event() for _ in range(self.n_chunk_slots)]
        for ev in self.slot_free_events:
            ev.record(compute)
        self.spares = []
        self._new_spare()
        self.n_units = self.num_stream * self.n_types
        self.unit_events = [None] * self.n_units
        self.scratch = None
        self.scratch_views = {}
        self.calibrating = False
        log_info(f"DiT Layer Streaming [chunks]: {self.n_types} chunks per block (largest {self.slot_bytes / 1024 ** 2:.1f}"
                 f" MB), {self.n_chunk_slots} slots + {len(self.spares)} spare.")

    def _new_spare(self):
        buf = torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
        ev = _native.Event()
        ev.record(self.compute_stream())
        self.spares.append((buf, ev, [self._views(buf, plan[1]) for plan in self.type_plan]))
        return len(self.spares) - 1

    # ---- chunked forwards
    def begin_forward(self):
        super().begin_forward()           # the previous forward has run on the GPU: its events are free
        for ev in self._retired:
            ev.close()
        self._retired = []
        self.blocks_started = 0
        self._fwd = {"t0": time.perf_counter(), "spares": 0, "outside": 0}
        if self.types is None:
            return
        n = self.n_units
        self.u_issued = [False] * n
        self.u_bound = [False] * n
        self.u_complete = [False] * n
        self.u_dead = [False] * n         # dropped for this forward: its layers, if called, go the outside way
        self.u_spare = {}                 # unit -> spare index
        self.u_done = [set() for _ in range(n)]
        self.next_issue = 0
        self.slot_owner = [None] * self.n_chunk_slots
        self.spare_owner = [None] * len(self.spares)

    def _issue(self, u, spare=None):
        """Copy unit u into its rotating slot (or spare ``spare``) on the copy stream, after the buffer's previous
        unit finished."""
        s, t = divmod(u, self.n_types)
        stream = self.prefetch_stream.handle
        if spare is None:
            k = u % self.n_chunk_slots
            buf, free = self.chunk_slots[k], self.slot_free_events[k]
            self.slot_owner[k] = u
        else:
            buf, free, _ = self.spares[spare]
            self.spare_owner[spare] = u
            self.u_spare[u] = spare
        if self.host_fence:
            free.synchronize()            # host-side fence (see leaf_pre)
        _native.stream_wait(stream, free)
        self._copy(s, self.type_plan[t][0], buf, stream)
        ev = _native.Event()
        ev.record(stream)
        ev.query()                        # submit now without blocking the host
        if self.unit_events[u] is not None:
            self._retired.append(self.unit_events[u])
        self.unit_events[u] = ev
        self.u_issued[u] = True

    def pump(self):
        """Issue units in order while the rotating slot's previous unit has finished."""
        while self.next_issue < self.n_units:
            u = self.next_issue
            if self.u_issued[u]:
                self.next_issue += 1
                continue
            owner = self.slot_owner[u % self.n_chunk_slots]
            if owner is not None and not self.u_complete[owner]:
                return
            self._issue(u)
            self.next_issue += 1

    def _free_spare(self):
        for i, owner in enumerate(self.spare_owner):
            if owner is None or self.u_complete[owner]:
                return i
        i = self._new_spare()
        self.spare_owner.append(None)
        return i

    def _complete(self, u):
        if self.u_complete[u]:
            return
        self.u_complete[u] = True
        if u in self.u_spare:
            ev = self.spares[self.u_spare[u]][1]
        elif self.u_issued[u]:
            ev = self.slot_free_events[u % self.n_chunk_slots]
        else:
            ev = None
        if ev is not None:
            ev.record(self.compute_stream())
            ev.query()
        self.pump()

    def _bind_outside(self, s, leaf):
        """A leaf called before any block of this forward started: its bytes into a buffer of its own, on the
        compute stream (WEIGHTFERRY_OUTSIDE_LEAF=0: the chunk pipeline starts there instead)."""
        runs, where, total = self.leaf_plan[leaf]
        if self.outside_buf is None or self.outside_buf.numel() < total:
            self.outside_buf = torch.empty(max(self.leaf_bytes.values()), dtype=torch.uint8, device=self.device)
        compute = self.compute_stream()
        if s in self.disk_index:
            self._staged_copy(s, runs, self.outside_buf, compute)
        else:
            self._copy(s, runs, self.outside_buf, compute)
        self._bind(s, self._views(self.outside_buf, where))
        self._fwd["outside"] += 1

    def _outside(self):
        return self.blocks_started == 0 and _env.get("WEIGHTFERRY_OUTSIDE_LEAF") != "0"

    def leaf_pre(self, module):
        if self.calibrating:
            self._calib_leaf_pre(module)
            return
        s, leaf = self.mod_info[id(module)]
        if self._outside():
            self._bind_outside(s, leaf)
            return
        t = self.type_of_leaf[leaf]
        u = s * self.n_types + t
        if self.u_dead[u]:
            self._bind_outside(s, leaf)
            return
        if self.u_bound[u]:
            return
        if not self.u_issued[u]:
            self.pump()
        if not self.u_issued[u]:
            self._issue(u, spare=self._free_spare())
            self.spare_uses += 1
            self._fwd["spares"] += 1
        views = (self.spares[self.u_spare[u]][2][t] if u in self.u_spare
                 else self.slot_type_views[u % self.n_chunk_slots][t])
        # the host-side fence on the copy (see host_fence): no cross-stream wait is ever pending when the compute
        # stream waits; the host runs at most the slots' depth ahead of the GPU, and the copies stay ahead of compute
        if self.host_fence:
            self.unit_events[u].synchronize()
        _native.stream_wait(self.compute_stream(), self.unit_events[u])
        self._bind(s, views)
        self.u_bound[u] = True

    def leaf_post(self, module):
        if self.calibrating or self._outside():
            return
        s, leaf = self.mod_info[id(module)]
        t = self.type_of_leaf[leaf]
        u = s * self.n_types + t
        if self.u_dead[u]:
            return
        self.u_done[u].add(leaf)
        if len(self.u_done[u]) == len(self.types[t]):
            self._complete(u)

    def block_pre(self, s):
        if self.calibrating:
            self.blocks_started += 1
            return
        # units of earlier blocks that were never copied (a caching wrapper skipped their block, or layers it does
        # not call) are dropped for this forward; those copied but not run free their slots
        for u in range(s * self.n_types):
            if not self.u_issued[u]:
                self.u_issued[u] = self.u_complete[u] = self.u_dead[u] = True
        for u in range(s * self.n_types):
            if not self.u_complete[u]:
                self._complete(u)
        if self.blocks_started == 0:
            self.pump()
        self.blocks_started += 1

    def block_post(self, s):
        if self.calibrating:
            return
        for t in range(self.n_types):
            u = s * self.n_types + t
            if self.u_issued[u]:
                self._complete(u)

    def prefetch_first_slots(self):
        if not self.calibrating:
            self.pump()

    def wrap_prefetch(self, slot_idx):
        return

    def end_forward(self):
        fwd = self._fwd
        if self.ring is not None:
            self._ring_release()
            if self._ring_next != 0:
                # the forward stopped before the SSD tier's last block: the ring restarts its cycle (it waits for
                # the copies out of its buffers itself)
                self.ring.resync()
                self._ring_next = 0
        if self.calibrating:
            self.finish_calibration()
        elif fwd is not None and _env.get("WEIGHTFERRY_CHUNK_LOG") == "1":
            log_info(f"DiT Layer Streaming [chunks]: forward {(time.perf_counter() - fwd['t0']) * 1000:.0f} ms (host), "
                     f"{fwd['spares']} chunks via a spare, {fwd['outside']} layer calls outside a block")
        super().end_forward()

    def _buffers(self):
        bufs = list(self.chunk_slots) + [b for b, _, _ in self.spares]
        if self.scratch is not None:
            bufs.append(self.scratch)
        if self.outside_buf is not None:
            bufs.append(self.outside_buf)
        return [(b.data_ptr(), b.data_ptr() + b.numel()) for b in bufs]

    def restore_rest_binding(self):
        ranges = self._buffers()
        for params, rest in zip(self.block_params, self.rest):
            for p, r in zip(params, rest):
                ptr = p.data.data_ptr()
                if any(a <= ptr < b for a, b in ranges):
                    p.data = r

    def close(self):
        if self.ring is not None and self._held is not None:
            self._ring_release()
        super().close()
        for e in getattr(self, "slot_free_events", []) + getattr(self, "unit_events", []) + self._retired:
            if e is not None:
                e.close()
        self._retired = []
        for _, ev, _ in self.spares:
            ev.close()
        if self._staging is not None and self._staging[1] is not None:
            self._staging[1].close()
        self._staging = None
        self.chunk_slots, self.spares = [], []
        self.scratch = self.outside_buf = None
