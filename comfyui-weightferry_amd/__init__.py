"""MI355X (gfx950) drop-in for WeightFerry's quantized-weight hot path.

Loaded by ComfyUI like the reference package (a custom-node directory; the directory name is the module name).
At import it installs the GGUF dequantisation patch when ComfyUI-GGUF is loaded, as the reference's package does
(__init__.py:94-95 of the reference), and registers the block-streaming node WeightFerryDiT under the reference's
name (__init__.py:104-132).

Sub-modules (the reference's names): enhancers.gguf_dequant, enhancers.fused_int8, enhancers.int8_block,
enhancers.fused_state, enhancers.fused_gguf (dequant + GEMM in one kernel), streaming.{common,state,profiler,
load_steps,dit_node,node}, core.tiers.{pinned,sources,plan,gguf_file}, core.env, utils.logging; the kernels live in
lib/libweightferry_hip.so
(csrc/, C ABI in include/weightferry.h).
"""

from .streaming.node import WeightFerryDiT  # noqa: E402

NODE_CLASS_MAPPINGS = {"WeightFerryDiT": WeightFerryDiT}
NODE_DISPLAY_NAME_MAPPINGS = {"WeightFerryDiT": "DiT Layer Streaming (low VRAM)"}


def _install_patches():
    from .utils.logging import log_warn
    try:
        from .enhancers import gguf_dequant
        gguf_dequant.install()
    except Exception as exc:  # noqa: BLE001 -- an import-time patch never breaks the host application
        log_warn(f"GGUF HIP dequant: not installed ({exc!r}).")


_install_patches()
