"""Opt-in stage timing, the analogue of hymm/utils/inference_metrics.py:139-156.

``stage(name)`` / ``@profiled(name)`` record wall time (with a device
synchronize on both sides) only while a ``StageMetrics`` collector is active;
otherwise they cost one attribute lookup.
"""
from __future__ import annotations

import contextlib
import functools
import time
from collections import defaultdict

_active = None


class StageMetrics:
    """Collects {stage name: [seconds, ...]} while used as a context manager."""

    def __init__(self, synchronize: bool = True):
        self.synchronize = synchronize
        self.samples = defaultdict(list)
        self._prev = None

    def __enter__(self):
        global _active
        self._prev, _active = _active, self
        return self

    def __exit__(self, *exc):
        global _active
        _active = self._prev
        return False

    def summary(self) -> dict:
        return {k: {"calls": len(v), "seconds": float(sum(v))} for k, v in self.samples.items()}


def _sync():
    import torch
    if torch.cuda.is_available():
        torch.cuda.synchronize()


@contextlib.contextmanager
def stage(name: str):
    m = _active
    if m is None:
        yield
        return
    if m.synchronize:
        _sync()
    t0 = time.perf_counter()
    try:
        yield
    finally:
        if m.synchronize:
            _sync()
        m.samples[name].append(time.perf_counter() - t0)


def profiled(name: str):
    def deco(fn):
        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            if _active is None:
                return fn(*args, **kwargs)
            with stage(name):
                return fn(*args, **kwargs)
        return wrapper
    return deco
