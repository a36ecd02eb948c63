"""The hot path's flags, with the reference's names and defaults (core/env.py:16-92 of the reference): an
environment variable overrides the default (core/env.py:130-135; the reference also reads a settings file in
ComfyUI's user directory, which is part of the host application and not of this path)."""
import os

DEFAULTS = {
    "WEIGHTFERRY_GGUF_TRITON": "1",        # GGUF dequantisation on the GPU kernel (the name is the reference's)
    "WEIGHTFERRY_GGUF_KQUANTS": "1",       # K-quants too
    "WEIGHTFERRY_GGUF_LORA_FACTORS": "pin",
    "WEIGHTFERRY_FUSED_BLOCK": "1",
    "WEIGHTFERRY_PROFILE": None,           # "1": per-block event timeline of block streaming
    "WEIGHTFERRY_SLOTS": None,             # number of GPU slots of block streaming (>= 2)
    # the reference's experimental prefetch-stream priority; every stream here keeps the default priority, so
    # the flag is read and ignored (streaming/state.py)
    "WEIGHTFERRY_PREFETCH_PRIORITY": None,
    # SSD tier
    "WEIGHTFERRY_TIERING": None,           # "auto" / "ram": overrides the node's tiering option
    "WEIGHTFERRY_RAM_BUDGET_GB": None,     # overrides the node's ram_budget_gb
    "WEIGHTFERRY_SSD_LAYOUT": None,        # "tail": the SSD tier is the last blocks (default: interleaved)
    "WEIGHTFERRY_MODEL_FILE": None,        # the GGUF file the SSD tier reads blocks from (else a cache file)
    "WEIGHTFERRY_CACHE_DIR": None,         # directory of the SSD tier's cache files (default: temp directory)
    "WEIGHTFERRY_RAM_MARGIN_GB": "6",      # RAM kept free besides the RAM tier when its budget is automatic
    "WEIGHTFERRY_DISK_THREADS": None,      # reader threads of the ring (default: the probe's fastest count)
    "WEIGHTFERRY_DISK_PROBE_MB": "512",    # size of the drive probe's scratch file
    "WEIGHTFERRY_PERSIST_GB": "0",         # > 0: keep SSD-tier cache files for later runs, this many GB at most
    # chunk (sub-block) streaming
    "WEIGHTFERRY_CHUNK": None,             # "1": the node streams chunks of blocks; "0" / unset: whole blocks
    "WEIGHTFERRY_CHUNK_MB": "96",          # bytes of layers per chunk
    "WEIGHTFERRY_CHUNK_SLOTS": "4",        # rotating chunk slots on the GPU (plus a spare)
    "WEIGHTFERRY_CHUNK_BLOCK0": "1",       # "0": block 0 stays resident in chunk mode
    "WEIGHTFERRY_CHUNK_RECALIBRATE": None,  # "1": learn the call order again on every load
    "WEIGHTFERRY_CHUNK_LOG": None,         # "1": a log line per chunked forward
    # "0" is refused: chunk streaming always keeps its host-side fences (streaming/chunk_state.py)
    "WEIGHTFERRY_CHUNK_HOST_FENCE": "1",
    "WEIGHTFERRY_OUTSIDE_LEAF": "1",       # "0": a layer called before any block starts the chunk pipeline
}


def get(name):
    if name in os.environ:
        return os.environ[name]
    return DEFAULTS.get(name)
