"""Deferred GPU-event timing of the attention stages.

Same contract as glob_set.queue_event_pair / resolve_latency_events (glob_set.py:32-66):
event pairs are queued while the forward runs and resolved after one synchronisation
into ``globVR.latency_stats[name] = {"time_ms": total, "calls": n}``.  Keys used by the
delta path: time_get_row_delta (select + pack + counts), time_delta_mm_pattern (hybrid
kernel), time_prefill_forward_total, time_triton_flash_attention.
"""
from __future__ import annotations

import torch

from . import globVR


def enabled() -> bool:
    """Stage timing is on (globVR.time_internal) and there is a device to time on."""
    return bool(getattr(globVR, "time_internal", False)) and torch.cuda.is_available()


def start_event():
    """Record and return a start event when timing is on, else None."""
    if not enabled():
        return None
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return ev


def stop_event(name: str, start) -> None:
    """Record the end event of ``start`` and queue the pair under ``name``."""
    if start is None:
        return
    end = torch.cuda.Event(enable_timing=True)
    end.record()
    queue_event_pair(name, start, end)


def queue_event_pair(metric_name: str, start_evt, end_evt) -> None:
    if not enabled():
        return
    if not hasattr(globVR, "latency_events"):
        globVR.latency_events = []
    globVR.latency_events.append((metric_name, start_evt, end_evt))


def resolve_latency_events() -> None:
    if not enabled() or not hasattr(globVR, "latency_events"):
        return
    if not hasattr(globVR, "latency_stats"):
        globVR.latency_stats = {}
    torch.cuda.synchronize()
    for name, s, e in globVR.latency_events:
        st = globVR.latency_stats.setdefault(name, {"time_ms": 0.0, "calls": 0})
        st["time_ms"] += s.elapsed_time(e)
        st["calls"] += 1
    globVR.latency_events.clear()


def reset() -> None:
    """Clear collected timings (eval_speedup.py:38-45)."""
    globVR.latency_stats = {}
    globVR.latency_events = []
    globVR.spars = 0.0
    globVR.kv_compression_samples = []
