"""Opt-in HIP-event timing of individual C-ABI launches.

``enable("glu_w1_forward")`` makes every later call of that op record a
start/end event pair on the stream it launches on; ``durations_ms(name)``
synchronises and returns the per-launch times. Disabled names cost one set
lookup per call.
"""

from __future__ import annotations

import contextlib

import torch

_enabled: set = set()
_events: dict = {}
_NULL = contextlib.nullcontext()


@contextlib.contextmanager
def _timed(name, dev):
    stream = torch.cuda.current_stream(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    try:
        yield
    finally:
        end.record(stream)
        _events.setdefault(name, []).append((start, end))


def region(name: str, dev):
    return _timed(name, dev) if name in _enabled else _NULL


def enable(*names: str) -> None:
    _enabled.update(names)


def disable(*names: str) -> None:
    if names:
        _enabled.difference_update(names)
    else:
        _enabled.clear()


def reset() -> None:
    _events.clear()


def durations_ms(name: str) -> list:
    pairs = _events.get(name, [])
    if pairs:
        pairs[-1][1].synchronize()
    return [s.elapsed_time(e) for s, e in pairs]
