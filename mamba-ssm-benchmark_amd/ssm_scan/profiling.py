"""Optional per-launch timing of the engine's entry points with HIP events.

Inside ``with KernelTimer() as t:`` every C-ABI launch made by this package is bracketed by
two events recorded on the stream the kernels are enqueued on (torch's current stream),
so ``t.times_ms()`` gives each entry point's device time per call.  Outside a timer nothing
is recorded and launches are not touched.
"""

import torch

_active = None


class KernelTimer:
    def __init__(self):
        self.records = {}

    def __enter__(self):
        global _active
        self._prev = _active
        _active = self
        return self

    def __exit__(self, *exc):
        global _active
        _active = self._prev
        return False

    def times_ms(self):
        torch.cuda.synchronize()
        return {k: [s.elapsed_time(e) for s, e in v] for k, v in self.records.items()}


def timed_launch(name, stream, fn):
    t = _active
    if t is None:
        return fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    rc = fn()
    end.record()
    t.records.setdefault(name, []).append((start, end))
    return rc
