"""Grid-coordinate events -> InputEvents (example/utils.py:60-80)."""
from __future__ import annotations

import numpy as np

from salt_amd.network import InputEvents


def grid_input_events(event_times, x, y, c, n_real_events, grid_shape) -> InputEvents:
    """source_idx = row-major index of (c, y, x) in grid_shape = (C, H, W); one sample or
    a batch.  Out-of-grid coordinates and invalid times raise ValueError."""
    source_idx = np.ravel_multi_index((np.asarray(c), np.asarray(y), np.asarray(x)),
                                      tuple(grid_shape))
    return InputEvents.checked(np.asarray(event_times), source_idx.astype(np.int32),
                               np.asarray(n_real_events))


def split_input_events(split, grid_shape) -> InputEvents:
    """A split's events as InputEvents with a leading sample axis."""
    return grid_input_events(split.event_times, split.x, split.y, split.c,
                             split.n_real_events, grid_shape)


def take_input_events(raw: InputEvents, idx) -> InputEvents:
    """Samples idx (index array or slice) of a batch."""
    return InputEvents(*(np.asarray(a)[idx] for a in raw))
