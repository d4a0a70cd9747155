"""Step-by-step trajectories of the integer forward (salt_core/trace.py): per neuron and
queue column, the register after the step, the step's spike, the event time and (the
integer path's addition) the step's overflow flag.  Produced by the trace kernel
(salt_layer_trace) through layer.forward(..., trace=True) / run_network(..., trace=True).
"""
from __future__ import annotations

from typing import NamedTuple, TypedDict

import numpy as np


class LayerForwardTrace(NamedTuple):
    """One layer's trajectories (salt_core/trace.py:13-22), shape (n, steps) per sample
    (leading batch axis when batched).  steps = max_queue_len for conv layers, the input
    stream length for FC layers."""
    spike_mask: object   # bool
    v_steps: object      # int32 register after each step (reset applied); last = v_final
    event_ms: object     # float32 time of the step's event; NaN past the real events
    overflowed: object   # bool, the value before write-back left the register's range


class TraceSummary(TypedDict):
    n: int
    steps: int
    total_spikes: int
    fired: np.ndarray
    idle_frac: float
    v_range: tuple[float, float]
    nonfinite_v: int


def summarize_trace_scalars(trace: LayerForwardTrace) -> TraceSummary:
    """One sample, one layer -> scalar summary (salt_core/trace.py:58-81)."""
    sm = np.asarray(_host(trace.spike_mask))
    vs = np.asarray(_host(trace.v_steps)).astype(np.float64)
    ms = np.asarray(_host(trace.event_ms))
    n, steps = sm.shape
    return {"n": n, "steps": steps, "total_spikes": int(sm.sum()),
            "fired": np.where(sm.sum(axis=1) > 0)[0],
            "idle_frac": float(np.isnan(ms).mean()),
            "v_range": (float(np.nanmin(vs)), float(np.nanmax(vs))),
            "nonfinite_v": int(np.sum(~np.isfinite(vs)))}


def _host(x):
    return x.detach().cpu().numpy() if hasattr(x, "detach") else x
