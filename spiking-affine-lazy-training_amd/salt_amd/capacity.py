"""Capacity knobs and per-layer diagnostics, as salt_core/capacity.py:13-63 defines them."""
from collections.abc import Iterator, Mapping
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
