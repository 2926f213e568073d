"""HIP-event region timing on the launching stream.

The MI355X counterpart of the reference's per-block CUDA-event timing
(workers/ditserve/models/wan/block.py:555-578, `block_cuda_ms`): a region
records a start and an end event on the current stream around the launches it
encloses, so the measured duration is GPU time of exactly those kernels.
Disabled profilers cost nothing; nothing here synchronises until summary().
"""
import collections
import contextlib

import torch


class EventProfiler:
    """`only`: names of the regions to time (None: all).  Each timed region costs
    two event records on the stream, which matters on short steps."""

    def __init__(self, enabled=True, only=None):
        self.enabled = enabled
        self.only = None if only is None else frozenset(only)
        self._events = collections.defaultdict(list)

    @contextlib.contextmanager
    def region(self, name):
        if not self.enabled or (self.only is not None and name not in self.only):
            yield
            return
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        try:
            yield
        finally:
            end.record()
            self._events[name].append((start, end))

    def reset(self):
        self._events.clear()

    def summary(self):
        """{region: {"count", "total_ms", "avg_ms"}} — synchronises."""
        torch.cuda.synchronize()
        out = {}
        for name, pairs in self._events.items():
            times = [s.elapsed_time(e) for s, e in pairs]
            out[name] = {"count": len(times), "total_ms": sum(times), "avg_ms": sum(times) / len(times)}
        return out


NULL = EventProfiler(enabled=False)
