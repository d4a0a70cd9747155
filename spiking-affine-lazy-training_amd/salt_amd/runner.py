"""NetworkRunner: a whole network's forward on the GPU with no host synchronisation
between layers -- the serving / benchmark form of Network.apply_batched.

Parameters are validated and uploaded once.  run() launches one salt_layer_forward per
layer on the current stream, chaining each layer's device-resident output stream into
the next.  Outputs are the per-layer spike streams, final registers and per-stream
statistics (min/max pre-write-back value, needed queue length, overflow), i.e. the
fields example/quant_run.py:71-103 reports.  Capacity overflow is detected afterwards
(check_fits); when a layer overflows, the exact reference truncation needs
Network.apply_batched (which re-runs that layer and cuts its stream as
salt_core/stream.py:49-64 does).
"""
from __future__ import annotations

import numpy as np
import torch

from salt_amd.quant.backend import QuantBackend, RawLayerOut, run_layer_kernel
from salt_amd.quant.fixed_point import RoundMode
from salt_amd.stream import EventStream


class NetworkRunner:
    def __init__(self, network, params, round_mode="round", device=None):
        self.network = network
        self.round_mode = RoundMode(round_mode)
        self.device = device or torch.device("cuda", torch.cuda.current_device())
        be = QuantBackend(round_mode=self.round_mode)
        self.dev_params = [be.device_params(l, p, self.device) for l, p in zip(network.layers, params)]

    def run(self, stream: EventStream, *, extremes: bool = False) -> list[RawLayerOut]:
        times = stream.event_times
        src = stream.event_source_idx
        n_real = stream.n_real_events.reshape(-1)
        outs = []
        last = len(self.network.layers) - 1
        for i, (layer, dp) in enumerate(zip(self.network.layers, self.dev_params)):
            out = run_layer_kernel(layer, dp, self.round_mode, times, src, n_real,
                                   int(layer.max_out_spikes), extremes=extremes,
                                   fill_pads=(i == last))
            outs.append(out)
            times, src, n_real = out.times, out.src, out.n
        return outs

    def check_fits(self, outs: list[RawLayerOut]) -> np.ndarray:
        """Per-stream fits (salt_core/network.py:116-121): every layer's spike count within
        max_out_spikes and, for conv layers, needed queue length within max_queue_len."""
        fits = None
        for layer, o in zip(self.network.layers, outs):
            f = o.n.cpu().numpy() <= layer.max_out_spikes
            if hasattr(layer, "max_queue_len"):
                f &= o.stats[:, 2].cpu().numpy() <= layer.max_queue_len
            fits = f if fits is None else fits & f
        return fits
