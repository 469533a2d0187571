"""Kernel timing inside real training steps.

``with timing.record() as rec: ...`` makes the library's autograd Functions bracket each HIP
library call with HIP events on the stream the call uses; ``rec.summary()`` (after the work
has completed) gives per-entry-point call counts and mean durations.  Outside such a block the
hook costs one attribute test per call.

Eager steps are launched from Python, and the GPU usually runs ahead of the host: without
care, the first event of a pair is processed as soon as the GPU reaches it, and the interval
then includes the time the GPU waits for the host to submit the call.  So each bracketed call
is queued behind a short spin kernel (``torch.cuda._sleep``, no memory traffic): while it
spins, the host enqueues the first event, the call and the second event, and the GPU then
executes them back to back.  What remains in the interval is the call's own kernels and two
event packets.
"""
from __future__ import annotations

import contextlib
from collections import defaultdict

import torch

_active = None

# Spin of the settle kernel in microseconds (converted to clock cycles on first use).
SETTLE_US = 60.0


class Recorder:
    def __init__(self, settle: bool = True, repeat: dict | None = None):
        self.events = defaultdict(list)
        self.settle = settle
        self.repeat = dict(repeat or {})
        self._cycles = None

    def settle_cycles(self) -> int:
        """Clock cycles of torch.cuda._sleep that spin for about SETTLE_US (measured once)."""
        if self._cycles is None:
            probe = 1_000_000
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(probe)       # warm-up
            a.record()
            torch.cuda._sleep(probe)
            b.record()
            b.synchronize()
            us = max(a.elapsed_time(b) * 1e3, 1e-3)
            self._cycles = max(1, int(probe * SETTLE_US / us))
        return self._cycles

    def summary(self) -> dict:
        """Per entry point: calls, and the mean duration of one launch (an interval around n
        repeated launches counts as n launches of interval / n each)."""
        torch.cuda.synchronize()
        out = {}
        for name, items in self.events.items():
            ms = [a.elapsed_time(b) / n for a, b, n in items]
            out[name] = {"calls": len(ms), "mean_ms": sum(ms) / len(ms),
                         "launches_per_interval": items[0][2]}
        return out


@contextlib.contextmanager
def record(settle: bool = True, repeat: dict | None = None):
    """Time the library calls made inside the block.  ``repeat`` maps entry-point names to a
    launch count n: such a call is issued n times back to back between its two events (the
    same arguments and outputs; only for calls that launch kernels into buffers allocated
    before the call, so that a repeat overwrites the same outputs with the same values)."""
    global _active
    prev, _active = _active, Recorder(settle, repeat)
    try:
        yield _active
    finally:
        _active = prev


def timed(name: str, fn, stream=None):
    """Run fn(); when a recorder is active, bracket it with events on `stream` (queued behind
    the settle spin, see the module docstring)."""
    rec = _active
    if rec is None:
        return fn()
    s = stream if stream is not None else torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = int(rec.repeat.get(name, 1))
    if rec.settle:
        cycles = rec.settle_cycles()
        with torch.cuda.stream(s):
            torch.cuda._sleep(cycles)
    a.record(s)
    r = fn()
    for _ in range(n - 1):
        fn()
    b.record(s)
    rec.events[name].append((a, b, n))
    return r
