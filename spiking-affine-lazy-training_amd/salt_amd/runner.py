"""NetworkRunner: a whole network's forward on the GPU with no host synchronisation
between layers -- the serving / benchmark form of Network.apply_batched.

Parameters are validated and uploaded once.  run() is one salt_network_forward call:
the library enqueues every layer on the current stream, each layer's device-resident
output stream feeding the next (run_network, salt_core/network.py:93-122).  run_layers()
does the same with one salt_layer_forward call per layer from Python, so that a caller
can bracket each layer's launch with HIP events.  Outputs are the per-layer spike
streams, final registers and per-stream statistics (min/max pre-write-back value,
needed queue length, overflow), i.e. the fields example/quant_run.py:71-103 reports.
Capacity overflow is detected afterwards (check_fits).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from salt_amd import _lib
from salt_amd.quant.backend import (QuantBackend, RawLayerOut, layer_desc, qparams,
                                    run_layer_kernel)
from salt_amd.quant.fixed_point import RoundMode
from salt_amd.stream import EventStream


def _alloc_out(layer, B: int, dev, extremes: bool) -> RawLayerOut:
    cap, n = int(layer.max_out_spikes), layer.n_neurons
    return RawLayerOut(
        times=torch.empty((B, cap), dtype=torch.float32, device=dev),
        src=torch.empty((B, cap), dtype=torch.int32, device=dev),
        n=torch.empty(B, dtype=torch.int32, device=dev),
        v_final=torch.empty((B, n), dtype=torch.int32, device=dev),
        v_min=torch.empty((B, n), dtype=torch.int32, device=dev) if extremes else None,
        v_max=torch.empty((B, n), dtype=torch.int32, device=dev) if extremes else None,
        stats=torch.empty((B, 4), dtype=torch.int32, device=dev))


class NetworkRunner:
    def __init__(self, network, params, round_mode="round", device=None):
        self.network = network
        self.round_mode = RoundMode(round_mode)
        self.device = device or torch.device("cuda", torch.cuda.current_device())
        be = QuantBackend(round_mode=self.round_mode)
        self.dev_params = [be.device_params(l, p, self.device) for l, p in zip(network.layers, params)]
        n = len(network.layers)
        # The descriptors point at dev_params' device buffers, which this object keeps.
        self._descs = (_lib.LayerDesc * n)(*[layer_desc(l) for l in network.layers])
        self._qps = (_lib.QParams * n)(*[qparams(dp, self.round_mode) for dp in self.dev_params])
        self._workspace: dict[tuple[int, int, bool], torch.Tensor] = {}

    def _workspace_for(self, B: int, L: int, extremes: bool) -> torch.Tensor:
        key = (B, L, extremes)
        ws = self._workspace.get(key)
        if ws is None:
            size = ctypes.c_size_t(0)
            _lib.check(_lib.lib().salt_network_workspace_size(
                len(self.network.layers), self._descs, self._qps, B, L, int(extremes),
                ctypes.byref(size)), "salt_network_workspace_size")
            ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device=self.device)
            self._workspace[key] = ws
        return ws

    def run(self, stream: EventStream, *, extremes: bool = False) -> list[RawLayerOut]:
        """Every layer in one salt_network_forward call; the last layer's stream has its
        pads filled (time 1e12, source 0) as the reference's output stream does."""
        times = stream.event_times.to(torch.float32).contiguous()
        src = stream.event_source_idx.to(torch.int32).contiguous()
        n_real = stream.n_real_events.reshape(-1).to(torch.int32).contiguous()
        B, L = times.shape
        layers = self.network.layers
        n = len(layers)
        last = n - 1
        outs = [_alloc_out(l, B, times.device, extremes) for l in layers]
        ws = self._workspace_for(B, L, extremes)
        ev_in = _lib.EventsIn(B=B, L=L, d_times=times.data_ptr(), d_src=src.data_ptr(),
                              d_n_real=n_real.data_ptr())
        ev_out = (_lib.EventsOut * n)(*[
            _lib.EventsOut(cap=int(l.max_out_spikes), d_times=o.times.data_ptr(),
                           d_src=o.src.data_ptr(), d_n=o.n.data_ptr(), fill_pads=int(i == last))
            for i, (l, o) in enumerate(zip(layers, outs))])
        res = (_lib.LayerResult * n)(*[
            _lib.LayerResult(d_v_final=o.v_final.data_ptr(), d_v_min=_lib.ptr(o.v_min),
                             d_v_max=_lib.ptr(o.v_max), d_stats=o.stats.data_ptr())
            for o in outs])
        _lib.check(_lib.lib().salt_network_forward(n, self._descs, self._qps,
                                                   ctypes.byref(ev_in), ev_out, res,
                                                   ws.data_ptr(), ws.numel(),
                                                   _lib.current_stream()),
                   "salt_network_forward")
        return outs

    def run_layers(self, stream: EventStream, *, extremes: bool = False,
                   around=None) -> list[RawLayerOut]:
        """One salt_layer_forward per layer.  around(i, phase) is called with phase 0
        before and 1 after layer i's launch (e.g. to record HIP events)."""
        times = stream.event_times
        src = stream.event_source_idx
        n_real = stream.n_real_events.reshape(-1)
        outs = []
        last = len(self.network.layers) - 1
        for i, (layer, dp) in enumerate(zip(self.network.layers, self.dev_params)):
            if around:
                around(i, 0)
            out = run_layer_kernel(layer, dp, self.round_mode, times, src, n_real,
                                   int(layer.max_out_spikes), extremes=extremes,
                                   fill_pads=(i == last))
            if around:
                around(i, 1)
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
