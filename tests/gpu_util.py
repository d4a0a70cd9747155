"""GPU-side helpers for the parity tests."""
import numpy as np
import torch

from salt_amd import EventStream, QuantBackend
from salt_amd.stream import unit_gain


def device_stream(times, src, n_real) -> EventStream:
    t = torch.from_numpy(np.ascontiguousarray(times, dtype=np.float32)).cuda()
    s = torch.from_numpy(np.ascontiguousarray(src, dtype=np.int32)).cuda()
    n = torch.from_numpy(np.ascontiguousarray(n_real, dtype=np.int32).reshape(-1)).cuda()
    return EventStream(t, s, unit_gain(t), n)


def run_layer(layer, params, times, src, n_real, round_mode="round", extremes=True):
    be = QuantBackend(round_mode=round_mode, neuron_extremes=extremes)
    out = layer.forward(params, device_stream(times, src, n_real), backend=be)
    torch.cuda.synchronize()
    return out
