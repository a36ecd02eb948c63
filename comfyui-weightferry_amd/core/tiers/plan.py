"""Tier planning: which streamed blocks the SSD tier serves (ssd_positions, core/tiers/plan.py:24-37 of the
reference), how many stay in RAM and how the reader ring is sized (plan_tiers, :60-150)."""
import math

from .. import env as _env


def ssd_positions(num_stream, n_disk, layout=None):
    """Streamed-block indices served from the SSD (ascending) for ``n_disk`` of ``num_stream`` blocks.

    "interleave" (default; WEIGHTFERRY_SSD_LAYOUT): spread evenly, the last block always on the SSD -- block k of
    the SSD tier is streamed block floor((k + 1) * num_stream / n_disk) - 1 -- so RAM-tier blocks compute between two
    SSD-tier blocks and the reader keeps reading with a small ring. "tail": the last n_disk blocks."""
    layout = layout or _env.get("WEIGHTFERRY_SSD_LAYOUT")
    if n_disk <= 0:
        return []
    if layout == "tail" or n_disk >= num_stream:
        return list(range(max(0, num_stream - n_disk), num_stream))
    return [(k + 1) * num_stream // n_disk - 1 for k in range(n_disk)]


def available_ram():
    """Available system RAM in bytes (psutil)."""
    import psutil
    return psutil.virtual_memory().available


def plan_tiers(num_stream, block_bytes, ram_budget_bytes=None, ram_margin_bytes=None, disk_gbps=None,
               compute_ms_per_block=None, disk_dir=None):
    """How many of ``num_stream`` streamed blocks of ``block_bytes`` stay in pinned RAM, and the SSD ring's depth and
    reader threads (plan_tiers, core/tiers/plan.py:60-150 of the reference, without its self-managed residents):
      * the budget is ``ram_budget_bytes``, or the available RAM minus a margin (WEIGHTFERRY_RAM_MARGIN_GB, 6 GB);
      * the drive's read rate is ``disk_gbps``, or what core.tiers.disk_io.probe_disk measures for ``disk_dir`` (with
        the thread count that read fastest; WEIGHTFERRY_DISK_THREADS overrides it);
      * the ring reads ahead enough to cover one block's read with block compute (+2), 2..8 buffers -- 4 without a
        read rate and a compute time -- and its pinned buffers count against the budget (fewer, down to 2, when the
        budget cannot hold them);
      * the rest of the budget holds whole blocks; the others go to the SSD tier.
    Returns {"ram_blocks", "disk_blocks", "ring_depth", "ring_threads", "budget", "ssd_bound", "disk_read_gbps",
    "disk_error"} (ssd_bound: reading the SSD tier takes longer than one forward's compute)."""
    if ram_budget_bytes is None:
        margin = ram_margin_bytes
        if margin is None:
            margin = int(float(_env.get("WEIGHTFERRY_RAM_MARGIN_GB") or 6.0) * 1024 ** 3)
        budget = max(0, available_ram() - margin)
    else:
        budget = max(0, int(ram_budget_bytes))
    out = {"budget": budget, "disk_read_gbps": disk_gbps, "disk_error": None, "ring_threads": 1}
    if budget >= num_stream * block_bytes:
        return dict(out, ram_blocks=num_stream, disk_blocks=0, ring_depth=0, ssd_bound=False)
    if disk_gbps is None and disk_dir is not None:
        from .disk_io import probe_disk
        try:
            probe = probe_disk(disk_dir, size_mb=int(_env.get("WEIGHTFERRY_DISK_PROBE_MB") or 512))
        except OSError as exc:            # no read rate: the plan falls back to the fixed depth
            out["disk_error"] = str(exc)
        else:
            threads = int(_env.get("WEIGHTFERRY_DISK_THREADS") or probe["threads"])
            disk_gbps = probe["by_threads"].get(threads, probe["gbps"])
            out.update(disk_read_gbps=disk_gbps, ring_threads=max(1, threads))
    depth = 4
    if disk_gbps and compute_ms_per_block:
        t_disk_ms = block_bytes / (disk_gbps * 1e9) * 1e3
        depth = max(2, min(8, math.ceil(t_disk_ms / compute_ms_per_block) + 2))
    while depth > 2 and depth * block_bytes > budget:
        depth -= 1
    ram_blocks = max(0, min(num_stream, (budget - depth * block_bytes) // block_bytes))
    disk = num_stream - ram_blocks
    ssd_bound = bool(disk_gbps and compute_ms_per_block
                     and disk * block_bytes / (disk_gbps * 1e9) * 1e3 > num_stream * compute_ms_per_block)
    return dict(out, ram_blocks=int(ram_blocks), disk_blocks=int(disk), ring_depth=depth, ssd_bound=ssd_bound)
