"""EventStream: the stream between layers, with the fields of salt_core/stream.py:16-21.

Arrays are torch tensors on the GPU: event_times float32 (integer ms), event_source_idx
int32, n_real_events int32, each with an optional leading batch axis.  The first
n_real_events entries are real, the rest are pads (time PAD_TIME, source 0, as
salt_core/stream.py:42-45 writes them).  The integer path gives every spike gain 1
(salt_core/quant/backend.py:52-53), so event_gain is a broadcast view of ones.
"""
from typing import NamedTuple

import torch

PAD_TIME = 1e12  # salt_core/stream.py:13


class EventStream(NamedTuple):
    event_times: torch.Tensor
    event_source_idx: torch.Tensor
    event_gain: torch.Tensor
    n_real_events: torch.Tensor


def unit_gain(event_times: torch.Tensor) -> torch.Tensor:
    """Gain 1 for every entry, as a zero-copy broadcast view."""
    return torch.ones(1, dtype=torch.float32, device=event_times.device).expand(event_times.shape)


def stream_hash(stream: EventStream) -> torch.Tensor:
    """Order-sensitive 64-bit hash of each stream of a batched EventStream, computed on
    the GPU (salt_stream_hash in libsalt_hip.so); returns int64 (B,) holding the bits.
    Used to compare streams too large to copy back."""
    from salt_amd import _lib
    t = stream.event_times.contiguous()
    s = stream.event_source_idx.to(torch.int32).contiguous()
    n = stream.n_real_events.reshape(-1).to(torch.int32).contiguous()
    B, cap = t.shape
    out = torch.empty(B, dtype=torch.int64, device=t.device)
    _lib.check(_lib.lib().salt_stream_hash(t.data_ptr(), s.data_ptr(), n.data_ptr(), B, cap,
                                           out.data_ptr(), _lib.current_stream()),
               "salt_stream_hash")
    return out
