"""Capacities of the layers (the knobs that size their queues and output streams), the
per-layer diagnostics a forward reports, and the rules that resize the knobs until every
sample fits -- the semantics of salt_core/capacity.py, whose knob names, policy fields
and results a model folder records.

A layer exposes `capacity` (a Capacity, or None) and `with_capacity(c)`; a diagnostic's
`needed` maps each knob to what one sample (or, per sample, a batch) required.  The
`max_extra_steps` knob only sizes the reference's float scan; it is carried and resized
with the same rule so that the capacities written to a model folder are the reference's.
"""
from __future__ import annotations

import math
from collections.abc import Iterator, Mapping, Sequence
from dataclasses import dataclass
from typing import NamedTuple

import torch


class LayerDiag(NamedTuple):
    """One layer's forward diagnostics: spike_count; firing_rate = spike_count /
    (n_neurons * max(real input events, 1)); needed: knob -> the capacity required
    (salt_core/capacity.py:13-22).  Per sample when the forward was batched."""
    spike_count: torch.Tensor
    firing_rate: torch.Tensor
    needed: dict


def reduce_over_batch(diag: LayerDiag) -> LayerDiag:
    """A batch's per-sample diagnostics as one: the means of the counts and the largest
    need per knob (one sample that does not fit means the batch does not)."""
    return LayerDiag(spike_count=torch.as_tensor(diag.spike_count).float().mean(),
                     firing_rate=torch.as_tensor(diag.firing_rate).float().mean(),
                     needed={knob: torch.as_tensor(need).max() for knob, need in diag.needed.items()})


class Capacity(Mapping):
    """An immutable knob -> capacity map (salt_core/capacity.py:35-63)."""

    __slots__ = ("_values",)

    def __init__(self, **knobs: int):
        self._values = {name: int(v) for name, v in knobs.items()}

    def __getitem__(self, knob: str) -> int:
        return self._values[knob]

    def __iter__(self) -> Iterator[str]:
        return iter(self._values)

    def __len__(self) -> int:
        return len(self._values)

    def __repr__(self) -> str:
        return "Capacity(" + ", ".join(f"{k}={v}" for k, v in self._values.items()) + ")"

    def replace(self, **knobs: int) -> Capacity:
        """A copy with some knobs set; a knob this capacity does not have raises KeyError."""
        missing = sorted(set(knobs).difference(self._values))
        if missing:
            raise KeyError(f"沒有這些旋鈕:{missing},有的是 {list(self._values)}")
        return Capacity(**(self._values | knobs))

    def fits(self, diag: LayerDiag) -> torch.Tensor:
        """Whether every knob holds what diag needed (per sample for a batch's diagnostics)."""
        ok = None
        for knob, value in self._values.items():
            holds = torch.as_tensor(diag.needed[knob]) <= value
            ok = holds if ok is None else ok & holds
        return ok


def _with_margin(need, factor: float) -> int:
    """The capacity granted for a need: ceil(need * factor)."""
    return int(math.ceil(int(need) * factor))


@dataclass(frozen=True)
class GrowthPolicy:
    """How one layer's knobs grow and shrink (salt_core/capacity.py:71-124).  A knob that
    is too small grows to ceil(need * factor); a knob with a shrink threshold drops to
    max(ceil(observed * factor), 1) once that is below value * threshold.  Growth and
    shrinking use the same factor, so an unchanged need maps to the same value both ways."""
    max_queue_len_grow_factor: float = 1.5
    out_grow_factor: float = 1.5
    max_extra_steps_grow_factor: float = 1.5
    out_shrink_threshold: float = 0.5
    max_extra_steps_shrink_threshold: float = 0.5

    def rule(self, knob: str) -> tuple[float, float | None]:
        """(grow factor, shrink threshold or None) of a knob."""
        return {"max_queue_len": (self.max_queue_len_grow_factor, None),
                "max_out_spikes": (self.out_grow_factor, self.out_shrink_threshold),
                "max_extra_steps": (self.max_extra_steps_grow_factor,
                                    self.max_extra_steps_shrink_threshold)}[knob]

    def grown(self, capacity: Capacity, needed: Mapping, chunk_size: int) -> Capacity:
        """Every knob that needed more than it holds, grown.  When max_queue_len grows,
        max_extra_steps becomes the value that always suffices for the new queue (the
        step need measured on a queue too short to hold the sample is not trusted)."""
        from salt_amd.layers.base import safe_extra_steps
        values = dict(capacity)
        for knob, value in capacity.items():
            if int(needed[knob]) > value:
                values[knob] = _with_margin(needed[knob], self.rule(knob)[0])
        if "max_extra_steps" in values and values.get("max_queue_len") != capacity.get("max_queue_len"):
            values["max_extra_steps"] = safe_extra_steps(values["max_queue_len"], chunk_size)
        return Capacity(**values)

    def shrunk(self, capacity: Capacity, observed: Mapping) -> Capacity:
        """Knobs with a shrink threshold reduced to what an epoch's largest needs
        (observed) call for, when that is well below their value; never below 1 (a layer
        that never fired would otherwise hand the next layer an empty input)."""
        values = dict(capacity)
        for knob, value in capacity.items():
            factor, threshold = self.rule(knob)
            if threshold is None:
                continue
            target = max(_with_margin(observed[knob], factor), 1)
            if target < value * threshold:
                values[knob] = target
        return Capacity(**values)


def _resized(layers: Sequence, capacities: Sequence) -> Sequence:
    """layers with each new capacity applied (None: keep); the very same sequence when no
    layer changed, so that callers can tell nothing was rebuilt."""
    out = list(layers)
    changed = False
    for i, (layer, cap) in enumerate(zip(layers, capacities)):
        if cap is not None and cap != layer.capacity:
            out[i] = layer.with_capacity(cap)
            changed = True
    return out if changed else layers


def grown_to_fit(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                 diags: Sequence[LayerDiag]) -> Sequence:
    """Each layer whose diagnostics (already reduced over the batch) did not fit, grown
    by its policy."""
    return _resized(layers, [
        None if layer.capacity is None
        else policies[layer.name].grown(layer.capacity, diag.needed, layer.chunk_size)
        for layer, diag in zip(layers, diags)])


def grown_to_fit_batch(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                       batch_diags: Sequence[LayerDiag]) -> Sequence:
    """grown_to_fit on per-sample diagnostics."""
    return grown_to_fit(layers, policies, [reduce_over_batch(d) for d in batch_diags])


def shrunk_to_observed(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                       observed: Mapping[str, Mapping[str, int]]) -> Sequence:
    """Each layer shrunk by its policy to the needs observed over an epoch (by name)."""
    return _resized(layers, [
        None if layer.capacity is None
        else policies[layer.name].shrunk(layer.capacity, observed[layer.name])
        for layer in layers])
