"""The WeightFerryDiT node: ComfyUI's entry to block streaming (streaming/dit_node.py:30-495 of the reference).

``WeightFerryDiT.apply_streaming(model, enabled, pin_memory, buffer_mode, resident_blocks, ...)`` keeps the
reference's signature, option names and choice strings (workflows store them). It clones the ModelPatcher and
registers
  * an ON_LOAD callback that, once ComfyUI has loaded and patched the weights (LoRA baked), captures the streamed
    blocks and installs the hooks (``dit_node.apply_streaming``) -- a later load tears the previous state down first;
  * an ON_DETACH callback that tears it down;
  * a DIFFUSION_MODEL wrapper that runs each forward with streaming active, capturing lazily when ComfyUI skipped
    ON_LOAD (a clone switch).
Block 0 stays resident (resident_blocks >= 1), as in the reference.

WEIGHTFERRY_CHUNK=1 streams chunks of blocks instead of whole blocks (streaming.chunk_state; the reference's
dit_node.py:215-246): the GPU holds WEIGHTFERRY_CHUNK_SLOTS chunks of WEIGHTFERRY_CHUNK_MB of layers, the call
order learned at the first load is kept with the node for later loads, and with resident_blocks <= 1 block 0
streams too (WEIGHTFERRY_CHUNK_BLOCK0=0 keeps it resident). Chunk mode needs Double Buffer (without it the node
streams whole blocks); with tiering Auto the chunks of SSD-tier blocks are copied out of the reader ring.

Tiering "Auto" puts the streamed blocks over the RAM budget (``ram_budget_gb``; 0: the available RAM minus
WEIGHTFERRY_RAM_MARGIN_GB, see core.tiers.plan.plan_tiers) on the SSD tier:
read straight from the GGUF model file named by WEIGHTFERRY_MODEL_FILE (ComfyUI-GGUF's loaded tensors do not carry
their file's path), or else from a cache file of their captured bytes (WEIGHTFERRY_CACHE_DIR; kept for later runs
with WEIGHTFERRY_PERSIST_GB > 0). The ring's depth and reader threads follow the drive's measured read rate
(core.tiers.disk_io.probe_disk, remembered for a week). resident_mode "Self-managed" keeps the resident blocks in GPU
buffers of the node's own, bound for each forward (dit_node._ResidentBuffers). Options of the reference that belong to
other paths -- SageAttention, fp8 storage format, auto-configuration, the VRAM budget -- are accepted and logged as not
applied; the node then streams as with their defaults."""
import math
import os

from ..core import env as _env
from ..utils.logging import log_info, log_warn
from . import dit_node
from .common import _blocks

_WRAPPER_KEY = "weightferry_dit"
_NODE_ATTR = "_weightferry_node_stream"

BUFFER_DOUBLE = "Double Buffer (Async Prefetch, Recommended)"
BUFFER_SINGLE = "Single Buffer (Synchronous)"
TIERING_RAM = "RAM (all streamed blocks pinned in RAM)"
TIERING_AUTO = "Auto (GPU / RAM / SSD)"
RESIDENT_MODE_COMFY = "ComfyUI (Dynamic VRAM)"
RESIDENT_MODE_SELF = "Self-managed (fixed on GPU)"
HOST_FORMAT_BAKED = "Compute dtype, LoRA baked (fast with LoRA)"
HOST_FORMAT_STORAGE = "Storage dtype (fp8), LoRA on GPU (half transfer)"


def _comfy():
    import comfy.model_management as mm
    import comfy.patcher_extension as pe
    return mm, pe


def _teardown(dit):
    """Undo a capture: the streamed parameters get host copies of their weights (ComfyUI's unloaded state)."""
    sm = getattr(dit, _NODE_ATTR, None)
    if sm is not None:
        sm.teardown(device="cpu")
        setattr(dit, _NODE_ATTR, None)


class WeightFerryDiT:
    """Layer streaming for a ComfyUI DiT: the blocks that do not stay resident stream from pinned RAM (or the GGUF
    file) into GPU slots while the model runs, each copy overlapped with the previous blocks' compute."""

    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "model": ("MODEL",),
                "enabled": ("BOOLEAN", {"default": True}),
                "pin_memory": ("BOOLEAN", {"default": True}),
                "buffer_mode": ([BUFFER_DOUBLE, BUFFER_SINGLE], {"default": BUFFER_DOUBLE}),
                "resident_blocks": ("INT", {"default": 8, "min": 1, "max": 128, "step": 1}),
                "sage_attention": ("BOOLEAN", {"default": False}),
            },
            "optional": {
                "host_format": ([HOST_FORMAT_BAKED, HOST_FORMAT_STORAGE], {"default": HOST_FORMAT_BAKED}),
                "tiering": ([TIERING_RAM, TIERING_AUTO], {"default": TIERING_RAM}),
                "ram_budget_gb": ("FLOAT", {"default": 0.0, "min": 0.0, "max": 512.0, "step": 0.5}),
                "resident_mode": ([RESIDENT_MODE_COMFY, RESIDENT_MODE_SELF], {"default": RESIDENT_MODE_COMFY}),
                "sage_pv_fp16": ("BOOLEAN", {"default": False}),
                "auto_config": ("BOOLEAN", {"default": True}),
                "prefetch_slots": ("INT", {"default": 3, "min": 2, "max": 6, "step": 1}),
                "vram_budget_gb": ("FLOAT", {"default": 0.0, "min": 0.0, "max": 512.0, "step": 0.5}),
            },
        }

    RETURN_TYPES = ("MODEL",)
    RETURN_NAMES = ("model",)
    FUNCTION = "apply_streaming"
    CATEGORY = "WeightFerry/streaming"
    TITLE = "DiT Layer Streaming (low VRAM)"

    def apply_streaming(self, model, enabled: bool = True, pin_memory: bool = True, buffer_mode: str = BUFFER_DOUBLE,
                        resident_blocks: int = 8, sage_attention: bool = False, host_format: str = HOST_FORMAT_BAKED,
                        prefetch_slots: int = 3, resident_mode: str = RESIDENT_MODE_COMFY, tiering: str = TIERING_RAM,
                        ram_budget_gb: float = 0.0, auto_config: bool = False, sage_pv_fp16: bool = False,
                        vram_budget_gb: float = 0.0, _root=None, _key_prefix=None, _text_encoder=False):
        if not enabled:
            log_info("DiT Layer Streaming: Disabled, passing original model.")
            return (model,)
        mm, pe = _comfy()
        not_applied = [name for name, on in (
            ("sage_attention", sage_attention), ("sage_pv_fp16", sage_pv_fp16),
            ("host_format=storage", host_format == HOST_FORMAT_STORAGE),
            ("auto_config", auto_config),
            ("vram_budget_gb", bool(vram_budget_gb)), ("text encoder streaming", _text_encoder)) if on]
        if not_applied:
            log_info(f"DiT Layer Streaming: not part of this package, not applied: {', '.join(not_applied)}.")
        if _text_encoder:
            return (model,)
        patcher = model.clone()
        dit = _root if _root is not None else getattr(patcher.model, "diffusion_model", None)
        if dit is None:
            log_warn("DiT Layer Streaming: Model has no 'diffusion_model', skipping.")
            return (model,)
        if not mm.is_device_cuda(patcher.load_device):
            log_warn("DiT Layer Streaming: Device is not CUDA, skipping.")
            return (patcher,)
        blocks = _blocks(dit)
        if len(blocks) == 0:
            log_warn(f"DiT Layer Streaming: no transformer block list on {type(dit).__name__}, skipping.")
            return (patcher,)
        double = buffer_mode != BUFFER_SINGLE
        env_tier = _env.get("WEIGHTFERRY_TIERING")
        tier_auto = (env_tier == "auto") if env_tier else tiering == TIERING_AUTO
        chunk = _env.get("WEIGHTFERRY_CHUNK") == "1"
        if chunk and not double:
            log_info("DiT Layer Streaming [chunks]: chunk streaming needs Double Buffer; streaming whole blocks.")
            chunk = False
        # chunk mode streams block 0 as well when it has the other blocks' layout (the reference's stream_block0)
        uniform0 = len(blocks) > 1 and [(tuple(p.shape), p.dtype) for p in blocks[0].parameters()] == \
            [(tuple(p.shape), p.dtype) for p in blocks[1].parameters()]
        stream_block0 = (chunk and uniform0 and int(resident_blocks) <= 1
                         and _env.get("WEIGHTFERRY_CHUNK_BLOCK0") != "0")
        resident_k = 0 if stream_block0 else max(1, min(len(blocks), int(resident_blocks)))
        num_stream = len(blocks) - resident_k
        if num_stream <= 0:
            log_info("DiT Layer Streaming: All blocks resident, no streaming offload registered.")
            return (patcher,)
        order_cache = {}                      # the learned chunk call order, kept with this node for later loads
        env_budget = _env.get("WEIGHTFERRY_RAM_BUDGET_GB")
        budget = float(env_budget) if env_budget else float(ram_budget_gb)
        model_file = _env.get("WEIGHTFERRY_MODEL_FILE") if tier_auto else None
        owner = object()
        log_info(f"DiT Layer Streaming: Registering Late Offload ({resident_k}/{len(blocks)} resident, {num_stream} "
                 f"streaming blocks, pin_memory={pin_memory}, double_buffer={double}, "
                 f"prefetch_slots={prefetch_slots if double else 1}, tiering={'auto' if tier_auto else 'ram'}"
                 f"{', chunks' if chunk else ''})...")

        def on_load(p, device_to, lowvram_model_memory, force_patch_weights, full_load):
            dev = device_to if device_to is not None else p.load_device
            if not mm.is_device_cuda(dev):
                return
            _teardown(dit)                    # a previous capture of this model (or another config's)
            ram_blocks, depth, threads = None, 2, 2
            if tier_auto:
                from ..core.tiers.cache_files import default_cache_dir
                from ..core.tiers.plan import plan_tiers
                per = sum(q.numel() * q.element_size() for q in blocks[resident_k].parameters())
                # the drive the SSD tier reads: the model file's, or the cache file's
                disk_dir = os.path.dirname(os.path.abspath(model_file)) if model_file else default_cache_dir()
                plan = plan_tiers(num_stream, per, ram_budget_bytes=int(budget * 1024 ** 3) if budget > 0 else None,
                                  disk_dir=disk_dir)
                ram_blocks, depth, threads = plan["ram_blocks"], max(2, plan["ring_depth"]), plan["ring_threads"]
                rate = plan["disk_read_gbps"]
                log_info(f"DiT Layer Streaming [tiers]: RAM budget {plan['budget'] / 1024 ** 3:.1f} GB: "
                         f"{plan['ram_blocks']} blocks in RAM, {plan['disk_blocks']} on the SSD tier"
                         + (f" (ring of {plan['ring_depth']}, {threads} readers"
                            + (f", drive {rate:.1f} GB/s)." if rate else ").") if plan["disk_blocks"] else "."))
            sm = dit_node.apply_streaming(dit, device=dev, resident_blocks=resident_k, prefetch_slots=prefetch_slots,
                                          pin_memory=pin_memory, model_file=model_file or None, ram_blocks=ram_blocks,
                                          double_buffer=double or (ram_blocks is not None and ram_blocks < num_stream),
                                          ring_depth=depth, ring_threads=threads, chunk=chunk,
                                          order_cache=order_cache if chunk else None,
                                          self_resident=resident_mode == RESIDENT_MODE_SELF)
            sm.owner_node = owner
            setattr(dit, _NODE_ATTR, sm)
            n_ssd = len(sm.state.disk_index)
            src = model_file or (sm.state.disk_store.path if sm.state.disk_store is not None else "?")
            how = ", streamed in chunks" if chunk else ""
            log_info(f"DiT Layer Streaming [Late Offload]: {num_stream} blocks offloaded ({num_stream - n_ssd} in "
                     f"pinned RAM, {n_ssd} read from {src}){how}." if n_ssd else
                     f"DiT Layer Streaming [Late Offload]: {num_stream} blocks offloaded to pinned RAM{how}.")

        def on_detach(p, unpatch_all=True, *args, **kwargs):
            sm = getattr(dit, _NODE_ATTR, None)
            if sm is not None and getattr(sm, "owner_node", None) is owner:
                _teardown(dit)

        def wrapper(executor, *args, **kwargs):
            sm = getattr(dit, _NODE_ATTR, None)
            if sm is None or getattr(sm, "owner_node", None) is not owner:
                # ComfyUI skipped ON_LOAD (switching back to a clone whose weights are in place): capture now
                on_load(patcher, patcher.load_device, 0, False, True)
                sm = getattr(dit, _NODE_ATTR, None)
                if sm is None:
                    return executor(*args, **kwargs)
                log_info("DiT Layer Streaming: ON_LOAD was skipped by ComfyUI; captured lazily at forward.")
            return sm.run(executor, *args, **kwargs)

        patcher.add_callback(pe.CallbacksMP.ON_LOAD, on_load)
        patcher.add_callback(pe.CallbacksMP.ON_DETACH, on_detach)
        wrappers = patcher.model_options.setdefault("transformer_options", {}).setdefault("wrappers", {})
        wrappers.setdefault(pe.WrappersMP.DIFFUSION_MODEL, {}).pop(_WRAPPER_KEY, None)
        pe.add_wrapper_with_key(pe.WrappersMP.DIFFUSION_MODEL, _WRAPPER_KEY, wrapper, patcher.model_options,
                                is_model_options=True)
        patcher._weightferry_stream_owner = owner
        log_info("DiT Layer Streaming: Hooked to ModelPatcher. Offload will activate upon model load.")
        return (patcher,)
