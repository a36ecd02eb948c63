"""Tier planning: which streamed blocks the SSD tier serves (ssd_positions, core/tiers/plan.py:24-37 of the
reference)."""
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
