"""Block streaming of a model's transformer blocks: set-up and the forward wrapper (the roles of
WeightFerryDiT.apply_streaming and streaming_diffusion_model_wrapper, streaming/dit_node.py:150-455 of the
reference), for a torch module whose blocks are a ModuleList named blocks / transformer_blocks / layers / block.

The reference attaches these to ComfyUI's ModelPatcher (ON_LOAD callback, diffusion-model wrapper); the host
application is not part of this path, so here they are plain calls: ``apply_streaming`` captures the blocks and
installs the hooks, ``StreamedModel.__call__`` runs one forward with streaming active, ``teardown`` undoes it."""
import torch

from .common import _ACTIVE_ATTR, _STATE_ATTR, _blocks, _flat_layout, _specs, _views
from .load_steps import (_build_chunk_state, _build_state, _install_block_stream_hooks, _install_chunk_hooks,
                         _install_first_block_hook, _install_resident_profile_hooks)


class _ResidentBuffers:
    """Self-managed resident blocks (the reference's resident_mode "Self-managed", streaming/state.py:91-106): each
    block's parameters are copied once into a GPU buffer of its own, in the streamed blocks' 256-byte aligned flat
    layout, and bound to it for each forward only; between forwards the parameters hold their own tensors again
    (``rest``). The host application's memory manager can then move, offload or rewrite those tensors without
    touching what the forwards read."""

    def __init__(self, blocks, device):
        self.blocks = list(blocks)
        self.rest = [[p.data for p in b.parameters()] for b in self.blocks]
        self.flats, self.views = [], []
        for b in self.blocks:
            specs = _specs(b)
            offsets, total = _flat_layout(specs)
            flat = torch.empty(total, dtype=torch.uint8, device=device)
            views = _views(flat, specs, offsets)
            for p, v in zip(b.parameters(), views):
                v.copy_(p.data)
            self.flats.append(flat)
            self.views.append(views)

    def bind(self):
        for b, views in zip(self.blocks, self.views):
            for p, v in zip(b.parameters(), views):
                p.data = v

    def unbind(self):
        for b, rest in zip(self.blocks, self.rest):
            for p, r in zip(b.parameters(), rest):
                p.data = r

    def release(self, device=None):
        """The parameters get their own tensors back (moved to ``device`` when given); the buffers are freed."""
        for b, rest in zip(self.blocks, self.rest):
            for p, r in zip(b.parameters(), rest):
                p.data = r if device is None else r.to(device)
        self.flats, self.views = [], []


class StreamedModel:
    """A model whose blocks stream from pinned host memory through GPU slots."""

    def __init__(self, dit, state, resident_idx, stream_idx, owner, residents=None):
        self.dit = dit
        self.state = state
        self.resident_idx = resident_idx
        self.stream_idx = stream_idx
        self.owner = owner
        self.residents = residents            # _ResidentBuffers of self-managed resident blocks, or None

    def __call__(self, *args, **kwargs):
        """One forward of the model with streaming active."""
        return self.run(self.dit, *args, **kwargs)

    def run(self, fn, *args, **kwargs):
        """fn(*args, **kwargs) -- the model's forward, or the host application's executor of it -- with streaming
        active (streaming_diffusion_model_wrapper, streaming/dit_node.py:414-455): begin_forward, the owner token,
        and the slot bindings undone afterwards whatever happens."""
        dit, state = self.dit, self.state
        setattr(dit, _ACTIVE_ATTR, self.owner)
        prof = state.profiler
        try:
            state.begin_forward()
            if self.residents is not None:
                self.residents.bind()
            if prof is not None:
                prof.begin_forward(state.compute_stream())
            return fn(*args, **kwargs)
        finally:
            if prof is not None:
                prof.end_forward(state.compute_stream())
            setattr(dit, _ACTIVE_ATTR, None)
            if self.residents is not None:
                self.residents.unbind()
            state.restore_rest_binding()
            state.end_forward()

    def profile_summary(self):
        return self.state.profile_summary()

    def teardown(self, device=None):
        """Move the streamed blocks' parameters back to ``device`` (default: the slots' device), release the pinned
        buffers and slots."""
        state = self.state
        dev = torch.device(device) if device is not None else state.device
        if self.residents is not None:
            self.residents.release(dev)
            self.residents = None
        state.close()
        for blk in state.streaming_blocks:
            for p in blk.parameters():
                p.data = p.data.to(dev, copy=True)
        for h in getattr(state, "holders", []):
            h.release()
        state.slot_flats = []
        state.slot_views = []
        if getattr(self.dit, _STATE_ATTR, None) is state:
            delattr(self.dit, _STATE_ATTR)


def apply_streaming(dit, device="cuda", resident_blocks=0, prefetch_slots=2, pin_memory=True, profile=None,
                    model_file=None, ram_blocks=None, ssd_layout=None, ring_depth=2, ring_threads=1, direct_io=True,
                    tensor_name=None, double_buffer=True, ssd_dir=None, chunk=False, chunk_bytes=None,
                    chunk_slots=None, order_cache=None, self_resident=False):
    """Stream all but the first ``resident_blocks`` blocks of ``dit`` (which stay where they are, on ``device``)
    through ``prefetch_slots`` (>= 2) GPU slots. The reference keeps block 0 resident by default
    (streaming/dit_node.py:237-267); here resident_blocks = 0 streams every block. ``self_resident``: the resident
    blocks are copied into GPU buffers of their own and bound to them for each forward only (_ResidentBuffers)
    instead of being moved to ``device``.

    SSD tier: with ``ram_blocks`` below the number of streamed blocks, only ``ram_blocks`` blocks are captured into
    pinned RAM; the others (spread by ``ssd_layout``, see core.tiers.plan.ssd_positions) are read from disk on every
    forward by a ring of ``ring_depth`` pinned buffers and ``ring_threads`` readers (O_DIRECT when ``direct_io``):
    straight from a GGUF ``model_file`` holding the blocks' tensors, or else from a cache file the capture writes
    into ``ssd_dir`` (default WEIGHTFERRY_CACHE_DIR / the temp directory). ``tensor_name(block_index,
    param_name)`` gives a parameter's tensor name in the model file (default "<block list>.<index>.<param name>",
    ComfyUI-GGUF's naming of a DiT's state dict).

    With WEIGHTFERRY_PERSIST_GB > 0 the cache file is kept for later loads with the same block bytes
    (core.tiers.cache_files.PersistentEntry).

    ``chunk``: sub-block streaming (streaming.chunk_state): the GPU holds ``chunk_slots`` chunks of at most
    ``chunk_bytes`` of a block's layers instead of whole blocks; the first forward learns the blocks' call order,
    kept in ``order_cache`` (a dict) when one is given. Double buffering only; the SSD tier as above."""
    blocks = list(_blocks(dit))
    if not blocks:
        raise ValueError("the model has no block list (blocks / transformer_blocks / layers / block)")
    device = torch.device(device)
    resident_idx = list(range(min(resident_blocks, len(blocks))))
    stream_idx = list(range(len(resident_idx), len(blocks)))
    if not stream_idx:
        raise ValueError("no block left to stream")
    residents = None
    if self_resident and resident_idx:
        residents = _ResidentBuffers([blocks[i] for i in resident_idx], device)
    else:
        for i in resident_idx:
            blocks[i].to(device)
    owner = object()
    ssd = _ssd_tier(dit, blocks, stream_idx, model_file, ram_blocks, ssd_layout, ring_depth, ring_threads, direct_io,
                    tensor_name, ssd_dir)
    if chunk:
        if not double_buffer:
            raise ValueError("chunk streaming is double-buffered")
        state = _build_chunk_state(owner, device, [blocks[i] for i in stream_idx], chunk_bytes, chunk_slots,
                                   pin_memory, order_cache, ssd)
        _install_first_block_hook(dit, blocks[0], state, owner)
        _install_chunk_hooks(dit, state, owner)
        setattr(dit, _STATE_ATTR, state)
        return StreamedModel(dit, state, resident_idx, stream_idx, owner, residents)
    state = _build_state(owner, device, [blocks[i] for i in stream_idx], prefetch_slots, pin_memory, profile, ssd,
                         double_buffer)
    _install_first_block_hook(dit, blocks[0], state, owner)
    _install_block_stream_hooks(dit, state, owner)
    _install_resident_profile_hooks(dit, blocks, resident_idx, state, owner)
    setattr(dit, _STATE_ATTR, state)
    return StreamedModel(dit, state, resident_idx, stream_idx, owner, residents)


def _ssd_tier(dit, blocks, stream_idx, model_file, ram_blocks, ssd_layout, ring_depth, ring_threads, direct_io,
              tensor_name, ssd_dir):
    """The SSD tier's description for the state builders, or None when every streamed block stays in RAM."""
    ssd = None
    if model_file is None and ram_blocks is not None and ram_blocks < len(stream_idx):
        from ..core.tiers.plan import ssd_positions
        ssd = {"positions": ssd_positions(len(stream_idx), len(stream_idx) - max(0, int(ram_blocks)), ssd_layout),
               "cache_dir": ssd_dir, "depth": ring_depth, "threads": ring_threads, "direct": direct_io}
    elif model_file is not None and ram_blocks is not None and ram_blocks < len(stream_idx):
        from ..core.tiers.plan import ssd_positions
        from ..core.tiers.sources import gguf_block_source
        from .common import _block_list_attr, _flat_layout, _specs
        attr = _block_list_attr(dit)
        name_of = tensor_name or (lambda i, p: f"{attr}.{i}.{p}")
        positions = ssd_positions(len(stream_idx), len(stream_idx) - max(0, int(ram_blocks)), ssd_layout)
        offsets, _ = _flat_layout(_specs(blocks[stream_idx[0]]))
        pnames = [n for n, _ in blocks[stream_idx[0]].named_parameters()]
        names = [[name_of(stream_idx[s], p) for p in pnames] for s in positions]
        source, sizes = gguf_block_source(model_file, names, offsets)
        want = [p.numel() * p.element_size() for p in blocks[stream_idx[0]].parameters()]
        if sizes != want:
            bad = next(i for i, (a, b) in enumerate(zip(sizes, want)) if a != b)
            raise ValueError(f"{model_file}: tensor {names[0][bad]} holds {sizes[bad]} bytes, the parameter "
                             f"{want[bad]}")
        ssd = {"positions": positions, "source": source, "depth": ring_depth, "threads": ring_threads,
               "direct": direct_io}
    return ssd
