"""GPU-timeline profile of block streaming (WEIGHTFERRY_PROFILE=1), on the library's HIP events.

Every measurement is a *span*: the time on the GPU between two events of one block, summed over the blocks of a
forward. The hooks record the events under fixed names; ``_SPANS`` says which pairs make which span:

=============  =================  ==========================================================================
span           events             what it measures
=============  =================  ==========================================================================
dma            dma0 -> dma1       the block's host -> GPU copy, on the copy stream
conversion     dma1 -> ready      work between the copy and the block being usable (none when the slot is
                                  the copy's target: ``ready`` is recorded with ``dma1``)
stall          wait0 -> start     the compute stream waiting for the block (the copy time left exposed)
compute        start -> end       the block's own compute
resident       r_start -> r_end   a block that is not streamed (kept on the GPU)
=============  =================  ==========================================================================

Two figures are defined as the reference defines them, so numbers from both compare (streaming/profiler.py:
100-103): the hidden fraction ``overlap_ratio = 1 - stall / (dma + conversion)`` clamped to [0, 1], and the copy
rate ``dma_gbps = host bytes per block * streamed blocks / dma time``. CPU-side marks (``mark``) are events on an
idle stream of their own: such an event completes as soon as the host issues it, which places host progress on
the GPU's clock.
"""
from dataclasses import dataclass, field
from statistics import fmean

from .. import _native

_SPANS = {"dma": ("dma0", "dma1"), "conversion": ("dma1", "ready"), "stall": ("wait0", "start"),
          "compute": ("start", "end")}
_RESIDENT_SPAN = ("r_start", "r_end")

# per-forward keys of summary() and the figure each reports (the reference's key names: scripts read them)
_REPORTED = ("forward_ms", "resident_compute_ms", "streamed_compute_ms", "compute_idle_ms", "dma_ms",
             "dequant_lora_ms", "stall_ms", "overlap_ratio", "dma_gbps", "cpu_hook_ms")


@dataclass
class _Forward:
    start: object
    end: object = None
    blocks: dict = field(default_factory=dict)     # streamed block index -> {event name: event}
    resident: dict = field(default_factory=dict)   # resident block index -> {event name: event}
    host_s: float = 0.0                            # host time spent inside the streaming hooks

    def span_ms(self, table, first, last):
        return sum(ev[first].elapsed_ms(ev[last]) for ev in table.values() if first in ev and last in ev)


def _hidden_fraction(stall_ms, transfer_ms):
    if transfer_ms <= 0:
        return None
    return min(1.0, max(0.0, 1.0 - stall_ms / transfer_ms))


def _copy_rate_gbps(block_bytes, blocks, dma_ms):
    return block_bytes * blocks / (dma_ms * 1e-3) / 1e9 if dma_ms > 0 else None


class _StreamProfiler:
    """Events of up to ``MAX_FORWARDS`` forwards of a streamed model with ``num_stream`` streamed blocks of
    ``host_bytes`` each (the reference's _StreamProfiler interface, streaming/profiler.py:9-134). ``is_double`` and
    ``no_staging`` are reported as given."""

    MAX_FORWARDS = 64

    def __init__(self, num_stream, host_bytes, is_double, no_staging=True):
        self.num_stream = num_stream
        self.host_bytes = host_bytes
        self.is_double = is_double
        self.no_staging = no_staging
        self.forwards = []
        self.cur = None
        # copies issued during one forward for the next one (the tail of a forward prefetches the next forward's
        # first blocks): their events belong to the forward that uses them
        self._early = {}
        self.marker_stream = _native.Stream()

    # ------------------------------------------------------------------------------------------ recording
    @staticmethod
    def _stamp(stream):
        ev = _native.Event(timing=True)
        ev.record(stream)
        return ev

    def begin_forward(self, stream):
        if len(self.forwards) >= self.MAX_FORWARDS:
            self.cur = None
            return
        self.cur = _Forward(start=self._stamp(stream), blocks=self._early)
        self._early = {}
        self.forwards.append(self.cur)

    def end_forward(self, stream):
        if self.cur is not None:
            self.cur.end = self._stamp(stream)
            self.cur = None

    def record(self, s_idx, name, stream, next_forward=False):
        """Event ``name`` of streamed block ``s_idx`` on ``stream`` (for the next forward when ``next_forward``)."""
        if next_forward:
            self._early.setdefault(s_idx, {})[name] = self._stamp(stream)
        elif self.cur is not None:
            self.cur.blocks.setdefault(s_idx, {})[name] = self._stamp(stream)

    def record_resident(self, b_idx, name, stream):
        """Event ``name`` ("r_start" / "r_end") of resident block ``b_idx`` on ``stream``."""
        if self.cur is not None:
            self.cur.resident.setdefault(b_idx, {})[name] = self._stamp(stream)

    def mark(self, s_idx, name):
        """The moment the host reaches this point, as an event of streamed block ``s_idx``."""
        if self.cur is not None:
            self.cur.blocks.setdefault(s_idx, {})[name] = self._stamp(self.marker_stream.handle)

    def add_cpu(self, seconds):
        if self.cur is not None:
            self.cur.host_s += seconds

    # ------------------------------------------------------------------------------------------- figures
    def _figures(self, f):
        spans = {name: f.span_ms(f.blocks, *ends) for name, ends in _SPANS.items()}
        resident_ms = f.span_ms(f.resident, *_RESIDENT_SPAN)
        total_ms = f.start.elapsed_ms(f.end)
        ratio = _hidden_fraction(spans["stall"], spans["dma"] + spans["conversion"])
        rate = _copy_rate_gbps(self.host_bytes, len(f.blocks), spans["dma"])
        return {
            "forward_ms": round(total_ms, 3),
            "streamed_blocks": len(f.blocks),
            "resident_compute_ms": round(resident_ms, 3),
            "streamed_compute_ms": round(spans["compute"], 3),
            # the compute stream running no block: stalls, gaps where the host was late, layers outside blocks
            "compute_idle_ms": round(total_ms - resident_ms - spans["compute"], 3),
            "dma_ms": round(spans["dma"], 3),
            "dequant_lora_ms": round(spans["conversion"], 3),
            "stall_ms": round(spans["stall"], 3),
            "overlap_ratio": None if ratio is None else round(ratio, 4),
            "dma_gbps": None if rate is None else round(rate, 2),
            "cpu_hook_ms": round(f.host_s * 1e3, 3),
        }

    def _timeline(self, f):
        """Every event of forward ``f`` in ms after its start: {"streamed": {block: {event: ms}}, "resident": ...}."""
        def table(blocks):
            return {str(b): {name: round(f.start.elapsed_ms(ev), 3) for name, ev in evs.items()}
                    for b, evs in sorted(blocks.items())}
        return {"forward_ms": round(f.start.elapsed_ms(f.end), 3), "streamed": table(f.blocks),
                "resident": table(f.resident)}

    def summary(self):
        """Per-forward figures, their mean over the forwards after the first (the first one also carries set-up
        costs), and the event timeline of one forward (the second, when there is one)."""
        done = [f for f in self.forwards if f.end is not None]
        if done:
            done[-1].end.synchronize()          # every earlier event is then complete as well
        per_forward = [self._figures(f) for f in done]
        steady = per_forward[1:] or per_forward
        mean = {}
        for key in _REPORTED:
            vals = [row[key] for row in steady if row[key] is not None]
            mean[key] = round(fmean(vals), 4) if vals else None
        return {
            "timeline_one_forward": self._timeline(done[min(1, len(done) - 1)]) if done else None,
            "forwards_recorded": len(per_forward),
            "host_mb_per_block": round(self.host_bytes / 2 ** 20, 1),
            "double_buffer": self.is_double,
            "storage_dtype_path": not self.no_staging,
            "mean_excluding_first_forward": mean,
            "per_forward": per_forward,
        }

    def close(self):
        self.forwards = []
        self._early = {}
        self.marker_stream.close()
