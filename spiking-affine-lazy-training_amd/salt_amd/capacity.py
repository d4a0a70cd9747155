"""Capacity knobs, per-layer diagnostics and the growth rules that enlarge a layer's
capacities until every sample fits, as salt_core/capacity.py defines them."""
import math
from collections.abc import Iterator, Mapping, Sequence
from dataclasses import dataclass
from typing import NamedTuple

import torch


class LayerDiag(NamedTuple):
    """spike_count, firing_rate = spike_count / (n_neurons * max(n_real_in, 1)) and
    needed: knob -> capacity this sample needs (salt_core/capacity.py:13-22)."""
    spike_count: torch.Tensor
    firing_rate: torch.Tensor
    needed: dict


def reduce_over_batch(diag: LayerDiag) -> LayerDiag:
    """Per-sample diagnostics of a batch -> one (salt_core/capacity.py:25-32)."""
    return LayerDiag(spike_count=diag.spike_count.float().mean(),
                     firing_rate=diag.firing_rate.float().mean(),
                     needed={k: torch.as_tensor(v).max() for k, v in diag.needed.items()})


class Capacity(Mapping):
    """Knob name -> capacity, immutable (salt_core/capacity.py:35-63)."""

    def __init__(self, **knobs: int):
        self._knobs = {k: int(v) for k, v in knobs.items()}

    def __getitem__(self, knob: str) -> int:
        return self._knobs[knob]

    def __iter__(self) -> Iterator[str]:
        return iter(self._knobs)

    def __len__(self) -> int:
        return len(self._knobs)

    def __repr__(self) -> str:
        return f"Capacity({', '.join(f'{k}={v}' for k, v in self._knobs.items())})"

    def replace(self, **knobs: int) -> "Capacity":
        unknown = set(knobs) - set(self._knobs)
        if unknown:
            raise KeyError(f"沒有這些旋鈕:{sorted(unknown)},有的是 {list(self._knobs)}")
        return Capacity(**{**self._knobs, **knobs})

    def fits(self, diag: LayerDiag) -> torch.Tensor:
        """Every knob holds diag.needed; per sample for batched diagnostics."""
        checks = [torch.as_tensor(diag.needed[k]) <= v for k, v in self._knobs.items()]
        return torch.stack(checks).all(dim=0)


def _grow(observed, factor: float) -> int:
    """ceil(observed * factor) (salt_core/capacity.py:66-68)."""
    return int(math.ceil(int(observed) * factor))


@dataclass(frozen=True)
class GrowthPolicy:
    """How one layer's capacities grow and shrink (salt_core/capacity.py:71-124).  Growing
    and shrinking share one factor per knob, so an unchanged need maps to the same value
    both ways."""
    max_queue_len_grow_factor: float = 1.5
    out_grow_factor: float = 1.5
    max_extra_steps_grow_factor: float = 1.5
    out_shrink_threshold: float = 0.5
    max_extra_steps_shrink_threshold: float = 0.5

    def _grow_factor(self, knob: str) -> float:
        return {"max_queue_len": self.max_queue_len_grow_factor,
                "max_out_spikes": self.out_grow_factor,
                "max_extra_steps": self.max_extra_steps_grow_factor}[knob]

    def _shrink_threshold(self, knob: str):
        return {"max_out_spikes": self.out_shrink_threshold,
                "max_extra_steps": self.max_extra_steps_shrink_threshold}.get(knob)

    def grown(self, capacity: Capacity, needed: Mapping, chunk_size: int) -> Capacity:
        """Knobs whose need exceeds their value grow to ceil(need * factor); a grown
        max_queue_len resets max_extra_steps to the value that always suffices."""
        from salt_amd.layers.base import safe_extra_steps
        new = {knob: _grow(needed[knob], self._grow_factor(knob))
               if int(needed[knob]) > value else value
               for knob, value in capacity.items()}
        if ("max_queue_len" in new and "max_extra_steps" in new
                and new["max_queue_len"] != capacity["max_queue_len"]):
            new["max_extra_steps"] = safe_extra_steps(new["max_queue_len"], chunk_size)
        return Capacity(**new)

    def shrunk(self, capacity: Capacity, observed: Mapping) -> Capacity:
        """Knobs with a shrink threshold drop to max(ceil(observed * factor), 1) when that
        is below value * threshold."""
        new = dict(capacity)
        for knob, value in capacity.items():
            threshold = self._shrink_threshold(knob)
            if threshold is None:
                continue
            candidate = max(_grow(observed[knob], self._grow_factor(knob)), 1)
            if candidate < value * threshold:
                new[knob] = candidate
        return Capacity(**new)


def _replace_capacity(layers: Sequence, new_capacities: Sequence) -> Sequence:
    """Layers whose capacity changed are replaced; the same list object comes back when
    none did (salt_core/capacity.py:142-150)."""
    replaced = [layer if cap is None or cap == layer.capacity else layer.with_capacity(cap)
                for layer, cap in zip(layers, new_capacities)]
    if all(new is old for new, old in zip(replaced, layers)):
        return layers
    return replaced


def grown_to_fit(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                 diags: Sequence[LayerDiag]) -> Sequence:
    """Layers that do not fit, grown; diags already reduced to scalars
    (salt_core/capacity.py:153-164)."""
    return _replace_capacity(layers, [
        None if layer.capacity is None
        else policies[layer.name].grown(layer.capacity, diag.needed, layer.chunk_size)
        for layer, diag in zip(layers, diags)])


def grown_to_fit_batch(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                       batch_diags: Sequence[LayerDiag]) -> Sequence:
    """grown_to_fit on per-sample diagnostics (salt_core/capacity.py:167-170)."""
    return grown_to_fit(layers, policies, [reduce_over_batch(d) for d in batch_diags])


def shrunk_to_observed(layers: Sequence, policies: Mapping[str, GrowthPolicy],
                       observed: Mapping[str, Mapping[str, int]]) -> Sequence:
    """salt_core/capacity.py:173-183."""
    return _replace_capacity(layers, [
        None if layer.capacity is None
        else policies[layer.name].shrunk(layer.capacity, observed[layer.name])
        for layer in layers])
