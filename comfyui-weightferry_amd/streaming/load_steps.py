"""Load-time steps of block streaming: capture of the streamed blocks into exact-size pinned host flats, the GPU
slots and the state, and the forward hooks -- the reference's streaming/load_steps.py on the direct path
(_capture_streamed_blocks :1152-1274, _build_state :719-766, _install_first_block_hook :315-337,
_install_block_stream_hooks :451-522)."""
import functools
import time

import torch

from .. import _native
from ..core import env as _env
from ..core.tiers.pinned import PinnedHost
from ..utils.logging import log_info
from .common import _ACTIVE_ATTR, _flat_layout, _specs, _views
from .profiler import _StreamProfiler
from .state import _StreamState


def _check_block_layouts(blocks):
    """Every streamed block must have the same parameter layout (one slot layout serves them all)."""
    specs = _specs(blocks[0])
    for i, blk in enumerate(blocks[1:], 1):
        if _specs(blk) != specs:
            raise ValueError(f"block {i} has a different parameter layout than block 0")
    return specs


def _capture_streamed_blocks(blocks, specs, offsets, flat_bytes, pin_memory=True, skip=()):
    """Copy each streamed block's parameters into its own flat host buffer (pinned when pin_memory); returns
    (holders, host_flats, host_views). Blocks whose index is in ``skip`` (the SSD tier's) get no host flat."""
    holders, host_flats, host_views = [], [], []
    for i, blk in enumerate(blocks):
        if i in skip:
            host_flats.append(None)
            host_views.append(None)
            continue
        if pin_memory:
            holder = PinnedHost(flat_bytes)
            holders.append(holder)
            flat = holder.tensor
        else:
            flat = torch.empty(flat_bytes, dtype=torch.uint8)
        flat.zero_()
        views = _views(flat, specs, offsets)
        for p, v in zip(blk.parameters(), views):
            v.copy_(p.data)
        host_flats.append(flat)
        host_views.append(views)
    return holders, host_flats, host_views


def _num_slots(prefetch_slots):
    n = max(2, int(prefetch_slots))
    if _env.get("WEIGHTFERRY_SLOTS"):
        n = max(2, int(_env.get("WEIGHTFERRY_SLOTS")))
    return n


def _ssd_cache(blocks, positions, specs, offsets, flat_bytes, ssd):
    """No model file to read: the SSD tier's blocks go into a cache file (their final bytes, as captured), or come
    from a persistent entry an earlier load wrote with the same content (WEIGHTFERRY_PERSIST_GB > 0). Returns (the
    ring's source, the store to delete at teardown or None)."""
    from ..core.tiers import cache_files as cf
    cap = float(_env.get("WEIGHTFERRY_PERSIST_GB") or 0) * 1024 ** 3
    entry = None
    if cap > 0:
        layout = ([(tuple(sh), str(dt)) for sh, dt in specs], list(offsets), int(flat_bytes), len(positions))
        key = cf.content_key(layout, (list(blocks[s].parameters()) for s in positions))
        entry = cf.PersistentEntry(cf.persistent_dir(ssd.get("cache_dir")), key, len(positions), flat_bytes)
        if entry.complete():
            log_info(f"DiT Layer Streaming [persist]: SSD cache reused ({entry.bin}).")
            return entry.source(), None
    store = (entry.open_store() if entry is not None
             else cf.DiskBlockStore(ssd.get("cache_dir") or cf.default_cache_dir(), flat_bytes, len(positions)))
    stage = torch.empty(flat_bytes, dtype=torch.uint8)
    views = _views(stage, specs, offsets)
    for k, s_idx in enumerate(positions):
        stage.zero_()
        for p, v in zip(blocks[s_idx].parameters(), views):
            v.copy_(p.data)
        store.write_block(k, stage)
    store.finalize()
    if entry is not None:
        freed = entry.commit(cap)
        log_info(f"DiT Layer Streaming [persist]: SSD cache kept for later runs ({entry.bin})"
                 + (f"; {freed / 1024 ** 3:.1f} GB of older entries removed." if freed else "."))
    return store.source(), store


def _rest_binding(blocks, host_views):
    """Bind each block's parameters to its host views; a block without (the SSD tier's) keeps its tensors. Returns
    the per-block tensors the parameters go back to between forwards."""
    rest = []
    for blk, views in zip(blocks, host_views):
        if views is None:
            rest.append([p.data for p in blk.parameters()])
            continue
        for p, v in zip(blk.parameters(), views):
            p.data = v
        rest.append(views)
    return rest


def _open_ring(blocks, positions, specs, offsets, flat_bytes, ssd, device):
    """The SSD tier's reader ring over its source (the model file's ranges, or a cache file written now): (ring,
    store to delete at teardown, source), or Nones without SSD-tier blocks."""
    if not positions:
        return None, None, None
    from ..core.tiers.sources import DiskRing
    source, store = ssd.get("source"), None
    if source is None:
        source, store = _ssd_cache(blocks, positions, specs, offsets, flat_bytes, ssd)
    if source.n_blocks != len(positions):
        raise ValueError(f"the SSD source has {source.n_blocks} blocks for {len(positions)} positions")
    if source.block_bytes > flat_bytes:
        raise ValueError(f"SSD-tier blocks of {source.block_bytes} bytes do not fit the {flat_bytes}-byte slots")
    ring = DiskRing(source, depth=int(ssd.get("depth", 2)), pin=True, threads=int(ssd.get("threads", 1)),
                    direct=bool(ssd.get("direct", True)), device=device)
    return ring, store, source


def _build_state(owner, device, blocks, prefetch_slots=2, pin_memory=True, profile=None, ssd=None, double_buffer=True):
    """Capture + slots + state for the given streamed blocks; the blocks' parameters end up bound to their host
    views (their "rest" tensors) until a forward binds them to a slot. ``ssd``: the SSD tier, a dict with
    "positions" (streamed-block indices it serves, ascending) and "source" (its blocks' file ranges in that order,
    see core.tiers.sources; each block's packed bytes in the flat layout) -- or, without a source, "cache_dir": the
    blocks' captured bytes are written into a cache file there (core.tiers.cache_files) -- optional "depth",
    "threads", "direct". Those blocks get no pinned host flat; their parameters keep their current tensors as rest binding (the
    reference's _setup_ssd_tier, streaming/load_steps.py:806-860). double_buffer=False: one slot, each block copied
    on the compute stream in its pre-hook (the reference's Single Buffer mode; not with an SSD tier)."""
    specs = _check_block_layouts(blocks)
    offsets, flat_bytes = _flat_layout(specs)
    positions = list((ssd or {}).get("positions") or [])
    holders, host_flats, host_views = _capture_streamed_blocks(blocks, specs, offsets, flat_bytes, pin_memory,
                                                               skip=set(positions))
    if not double_buffer and positions:
        raise ValueError("the SSD tier needs the double-buffered (prefetching) mode")
    num_slots = _num_slots(prefetch_slots) if double_buffer else 1
    slot_flats = [torch.empty(flat_bytes, dtype=torch.uint8, device=device) for _ in range(num_slots)]
    slot_views = [_views(f, specs, offsets) for f in slot_flats]
    rest = _rest_binding(blocks, host_views)
    ring, store, _ = _open_ring(blocks, positions, specs, offsets, flat_bytes, ssd, device)
    state = _StreamState(owner, device, list(blocks), host_flats, host_views, rest, slot_flats, slot_views,
                         is_double=double_buffer, ring=ring, disk_index={s: k for k, s in enumerate(positions)})
    state.disk_store = store
    state.holders = holders
    state.flat_bytes = flat_bytes
    if profile is None:
        profile = _env.get("WEIGHTFERRY_PROFILE") == "1"
    if profile:
        state.profiler = _StreamProfiler(len(blocks), flat_bytes, True, True)
    return state


def _build_chunk_state(owner, device, blocks, chunk_bytes=None, num_slots=None, pin_memory=True, order_cache=None,
                       ssd=None):
    """Capture + chunk streaming state (streaming/load_steps.py:736-753 of the reference): the blocks' host flats as
    for block streaming; the GPU holds ``num_slots`` chunk slots (WEIGHTFERRY_CHUNK_SLOTS, default 4) of at most
    ``chunk_bytes`` of layers each (WEIGHTFERRY_CHUNK_MB, default 96 MB) plus a spare, sized once the first forward
    has shown the blocks' call order. ``ssd``: the SSD tier as for _build_state; its blocks' chunks are copied out
    of the reader ring's buffers."""
    from .chunk_state import _ChunkState
    specs = _check_block_layouts(blocks)
    offsets, flat_bytes = _flat_layout(specs)
    positions = list((ssd or {}).get("positions") or [])
    holders, host_flats, host_views = _capture_streamed_blocks(blocks, specs, offsets, flat_bytes, pin_memory,
                                                               skip=set(positions))
    rest = _rest_binding(blocks, host_views)
    ring, store, source = _open_ring(blocks, positions, specs, offsets, flat_bytes, ssd, device)
    if chunk_bytes is None:
        chunk_bytes = int(float(_env.get("WEIGHTFERRY_CHUNK_MB")) * 1024 ** 2)
    if num_slots is None:
        num_slots = int(_env.get("WEIGHTFERRY_CHUNK_SLOTS"))
    state = _ChunkState(owner, device, list(blocks), host_flats, host_views, rest, specs, offsets, chunk_bytes,
                        num_slots, order_cache, ring=ring, disk_index={s: k for k, s in enumerate(positions)},
                        source=source)
    state.holders = holders
    state.flat_bytes = flat_bytes
    state.disk_store = store
    return state


def _install_chunk_hooks(dit, state, owner):
    """Chunk streaming: pre / post hooks on every streamed block and on each of its leaf modules
    (streaming/load_steps.py:359-397); block hooks first, so a block that owns parameters itself starts before its
    own leaf hook runs."""
    def make_block_hooks(cur_s):
        def block_pre(module, args):
            if getattr(dit, _ACTIVE_ATTR, None) is owner:
                state.block_pre(cur_s)

        def block_post(module, args, output):
            if getattr(dit, _ACTIVE_ATTR, None) is owner:
                state.block_post(cur_s)
        return block_pre, block_post

    def leaf_pre(module, args):
        if getattr(dit, _ACTIVE_ATTR, None) is owner:
            state.leaf_pre(module)

    def leaf_post(module, args, output):
        if getattr(dit, _ACTIVE_ATTR, None) is owner:
            state.leaf_post(module)

    for s_idx, blk in enumerate(state.streaming_blocks):
        pre_h, post_h = make_block_hooks(s_idx)
        state.handles.append(blk.register_forward_pre_hook(pre_h))
        state.handles.append(blk.register_forward_hook(post_h))
        for leaf_mod in state.leaf_modules[s_idx].values():
            state.handles.append(leaf_mod.register_forward_pre_hook(leaf_pre))
            state.handles.append(leaf_mod.register_forward_hook(leaf_post))


def _install_first_block_hook(dit, first_block, state, owner):
    """Pre-hook of the model's first block: the prefetch of the first slots, only when block 0 really runs."""
    def first_block_pre_hook(module, args):
        if getattr(dit, _ACTIVE_ATTR, None) is owner:
            t0 = time.perf_counter()
            state.prefetch_first_slots()
            if state.profiler is not None:
                state.profiler.add_cpu(time.perf_counter() - t0)
    state.handles.append(first_block.register_forward_pre_hook(first_block_pre_hook))


class _SlotHooks:
    """The per-block side of double buffering. Before streamed block s runs, the compute stream must not start it
    until its bytes are in its slot: reissue its copy if a skipped block broke the chain of prefetches, wait for the
    copy's event (on the host too, see ``_StreamState.host_fence``, then on the compute stream) and point the
    block's parameters at the slot. After it runs, the slot is free once the compute stream passes this point: record
    that, and start the copy of the block that takes the slot next (in this forward, or the next forward's first
    blocks when this was the slot's last one). The single-buffer mode copies on the compute stream instead."""

    def __init__(self, dit, state, owner):
        self.dit, self.state, self.owner = dit, state, owner

    def _ours(self):
        return getattr(self.dit, _ACTIVE_ATTR, None) is self.owner

    def _await_copy(self, s, compute, prof):
        st = self.state
        if not st.issued[s]:
            st.issue_prefetch(s)
        st.wait_transfer(s)
        landed = st.transferred_events[s]
        if prof is not None:
            prof.record(s, "wait0", compute)     # before the host fence: the GPU's idle time counts as stall
        if st.host_fence:
            landed.synchronize()
        _native.stream_wait(compute, landed)

    def before(self, s, module, args):
        if not self._ours():
            return
        st = self.state
        tic = time.perf_counter()
        prof, compute = st.profiler, st.compute_stream()
        if prof is not None:
            prof.mark(s, "cpu_pre_hook")
        if st.is_double:
            self._await_copy(s, compute, prof)
        else:
            if prof is not None:
                prof.record(s, "wait0", compute)
            st.materialize(s, 0, compute)
        if prof is not None:
            prof.record(s, "start", compute)
        for param, view in zip(module.parameters(), st.slot_views[st.slot_of(s)]):
            param.data = view
        if prof is not None:
            prof.add_cpu(time.perf_counter() - tic)

    def after(self, s, module, args, output):
        if not self._ours():
            return
        st = self.state
        prof, compute = st.profiler, st.compute_stream()
        if prof is not None:
            prof.record(s, "end", compute)
        if not st.is_double:
            return
        tic = time.perf_counter()
        slot = st.slot_of(s)
        st.computed_events[slot].record(compute)
        heir = s + st.num_slots                  # the next block to use this slot
        if heir >= st.num_stream:
            st.wrap_prefetch(slot)
        elif not st.issued[heir]:
            st.issue_prefetch(heir)
        if prof is not None:
            prof.add_cpu(time.perf_counter() - tic)


def _install_block_stream_hooks(dit, state, owner):
    """Registers _SlotHooks.before / after on every streamed block."""
    hooks = _SlotHooks(dit, state, owner)
    for s, blk in enumerate(state.streaming_blocks):
        state.handles.append(blk.register_forward_pre_hook(functools.partial(hooks.before, s)))
        state.handles.append(blk.register_forward_hook(functools.partial(hooks.after, s)))


def _install_resident_profile_hooks(dit, blocks, resident_idx, state, owner):
    """Blocks kept on the GPU (not streamed): r_start / r_end events on the compute stream when the profiler is on,
    so its summary separates their compute from the streamed blocks' and from idle time (the reference records
    them in its resident-block hooks, streaming/profiler.py:59-61)."""
    def make(b_idx):
        def pre(module, args):
            if state.profiler is not None and getattr(dit, _ACTIVE_ATTR, None) is owner:
                state.profiler.record_resident(b_idx, "r_start", state.compute_stream())

        def post(module, args, output):
            if state.profiler is not None and getattr(dit, _ACTIVE_ATTR, None) is owner:
                state.profiler.record_resident(b_idx, "r_end", state.compute_stream())
        return pre, post

    for b_idx in resident_idx:
        pre, post = make(b_idx)
        state.handles.append(blocks[b_idx].register_forward_pre_hook(pre))
        state.handles.append(blocks[b_idx].register_forward_hook(post))
