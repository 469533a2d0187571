"""Kernel timing inside real training steps.

``with timing.record() as rec: ...`` makes the library's autograd Functions bracket each HIP
library call with HIP events on the stream the call uses; ``rec.summary()`` (after the work
has completed) gives per-entry-point call counts and mean durations.  Outside such a block the
hook costs one attribute test per call.
"""
from __future__ import annotations

import contextlib
from collections import defaultdict

import torch

_active = None


class Recorder:
    def __init__(self):
        self.events = defaultdict(list)

    def summary(self) -> dict:
        torch.cuda.synchronize()
        out = {}
        for name, pairs in self.events.items():
            ms = [a.elapsed_time(b) for a, b in pairs]
            out[name] = {"calls": len(ms), "mean_ms": sum(ms) / len(ms)}
        return out


@contextlib.contextmanager
def record():
    global _active
    prev, _active = _active, Recorder()
    try:
        yield _active
    finally:
        _active = prev


def timed(name: str, fn, stream=None):
    """Run fn(); when a recorder is active, bracket it with events on `stream`."""
    rec = _active
    if rec is None:
        return fn()
    s = stream if stream is not None else torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    r = fn()
    b.record(s)
    rec.events[name].append((a, b))
    return r
