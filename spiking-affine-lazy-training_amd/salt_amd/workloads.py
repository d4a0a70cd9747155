"""Seeded synthetic workloads for the five benchmark configurations (host numpy).

Each builder returns a Workload: the Network, one QuantizedLayerParams per layer and a
padded batch of input events.  Unspecified quantisation settings are fixed as
f_a = 10, f_V = 0, i_V = 24, round, wrap, with decay tables from build_decay_table_int.
Randomness: numpy PCG64, SeedSequence(1000 + config_id); streams use spawned children,
weights the first spawned child of a separate SeedSequence(2000 + config_id).
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np

from salt_amd.layers import ConvLayer, FCLayer
from salt_amd.network import InputEvents, Network
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.quant.params import QuantizedLayerParams

F_A, F_V, I_V = 10, 0, 24


class Workload(NamedTuple):
    name: str
    network: Network
    params: list
    events: InputEvents      # numpy: times float32 (B, L), src int32 (B, L), n_real int32 (B,)
    round_mode: str


def _params(q, tau, v_th, overflow_mode="wrap", f_a=F_A, f_V=F_V, i_V=I_V):
    return QuantizedLayerParams(q=q, decay_table_int=build_decay_table_int(f_a, tau),
                                v_th_int=None if v_th is None else np.int32(v_th),
                                scale=np.float32(1.0), f_a=f_a, f_V=f_V, i_V=i_V,
                                overflow_mode=overflow_mode)


def _codes(rng, shape, sigma, bits):
    lim = 2 ** (bits - 1) - 1
    dt = np.int8 if bits == 8 else np.int16
    return np.clip(np.round(rng.normal(0.0, sigma, shape)), -lim, lim).astype(dt)


def _pad(streams, L=None):
    """List of (times, src) -> padded arrays; pads repeat the last time, source 0."""
    L = L or max(len(t) for t, _ in streams)
    B = len(streams)
    times = np.zeros((B, L), np.float32)
    src = np.zeros((B, L), np.int32)
    n_real = np.zeros(B, np.int32)
    for b, (t, s) in enumerate(streams):
        n = len(t)
        times[b, :n], src[b, :n], n_real[b] = t, s, n
        times[b, n:] = t[-1] if n else 0.0
    return InputEvents(times, src, n_real)


def blob_stream(rng, n_mean=4500, size=34, t_max=300, n_blobs=3):
    """Moving-blob events over a size x size x 2 plane: Poisson(n_mean) events, sorted
    integer times in [0, t_max), each from one of n_blobs blobs that move linearly from a
    random start in [4, size-5]^2 with velocity U(-0.08, 0.08) px/ms, position jittered by
    N(0, 2 px), polarity 50/50.  src = p*size*size + y*size + x."""
    n = int(rng.poisson(n_mean))
    t = np.sort(rng.integers(0, t_max, n)).astype(np.float32)
    start = rng.uniform(4, size - 5, (n_blobs, 2))
    vel = rng.uniform(-0.08, 0.08, (n_blobs, 2))
    which = rng.integers(0, n_blobs, n)
    pos = start[which] + vel[which] * t[:, None] + rng.normal(0.0, 2.0, (n, 2))
    pos = np.clip(np.round(pos), 0, size - 1).astype(np.int64)
    pol = rng.integers(0, 2, n)
    src = (pol * size * size + pos[:, 1] * size + pos[:, 0]).astype(np.int32)
    return t, src


def _children(config_id, B):
    return [np.random.default_rng(s) for s in np.random.SeedSequence(1000 + config_id).spawn(B)]


def _weight_rng(config_id):
    return np.random.default_rng(np.random.SeedSequence(2000 + config_id).spawn(1)[0])


def config1(B=1, n_events=4096) -> Workload:
    """FC 2312 -> 128, one stream of uniform events, times U{0..299}."""
    w = _weight_rng(1)
    layer = FCLayer(name="fc1", n_in=2312, n_out=128, init_k=1.0, tau=20.0, max_out_spikes=8192)
    params = [_params(_codes(w, (128, 2312), 24.0, 8), 20.0, 256)]
    streams = []
    for r in _children(1, B):
        streams.append((np.sort(r.integers(0, 300, n_events)).astype(np.float32),
                        r.integers(0, 2312, n_events).astype(np.int32)))
    return Workload("c1_fc2312x128", Network((2, 34, 34), [layer]), params, _pad(streams), "round")


def config2(B=256, n_mean=4500) -> Workload:
    """conv 2 -> 16, 5x5, s1, p0 on 34x34x2 (30x30x16 registers per stream)."""
    w = _weight_rng(2)
    streams = [blob_stream(r, n_mean) for r in _children(2, B)]
    ev = _pad(streams)
    layer = ConvLayer(name="conv1", ic=2, h_in=34, w_in=34, oc=16, k=5, s=1, p=0, init_k=1.0,
                      tau=20.0, max_queue_len=ev.event_times.shape[1] + 1, max_out_spikes=65536)
    params = [_params(_codes(w, (16, 2, 5, 5), 24.0, 8), 20.0, 128)]
    return Workload("c2_conv2x16k5", Network((2, 34, 34), [layer]), params, ev, "round")


def config3(B=1024, n_mean=4500, caps=(16384, 16384, 16384)) -> Workload:
    """N-MNIST-shaped net: conv(2->16, 5x5, s2) -> conv(16->32, 3x3, s2) -> FC(1568 -> 10)."""
    w = _weight_rng(3)
    streams = [blob_stream(r, n_mean) for r in _children(3, B)]
    ev = _pad(streams)
    L = ev.event_times.shape[1]
    c1 = ConvLayer(name="conv1", ic=2, h_in=34, w_in=34, oc=16, k=5, s=2, p=0, init_k=1.0,
                   tau=10.0, max_queue_len=L + 1, max_out_spikes=caps[0])
    c2 = ConvLayer(name="conv2", ic=16, h_in=15, w_in=15, oc=32, k=3, s=2, p=0, init_k=1.0,
                   tau=20.0, max_queue_len=caps[0] + 1, max_out_spikes=caps[1])
    out = FCLayer(name="out", n_in=32 * 7 * 7, n_out=10, init_k=1.0, tau=40.0,
                  max_out_spikes=caps[2])
    params = [_params(_codes(w, (16, 2, 5, 5), 24.0, 8), 10.0, 128),
              _params(_codes(w, (32, 16, 3, 3), 24.0, 8), 20.0, 128),
              _params(_codes(w, (10, 1568), 24.0, 8), 40.0, None)]
    return Workload("c3_nmnist_net", Network((2, 34, 34), [c1, c2, out]), params, ev, "round")


def config4(B=64, n_events=65536) -> Workload:
    """conv 2 -> 32, 3x3, s1 on 128x128x2 (126x126x32 registers per stream); the output
    capacity is the reference's default max_out_spikes (salt_core/layers/conv.py:50), far
    above the few spikes per stream this input gives."""
    w = _weight_rng(4)
    streams = []
    for r in _children(4, B):
        t = np.sort(r.integers(0, 2000, n_events)).astype(np.float32)
        x, y, p = r.integers(0, 128, n_events), r.integers(0, 128, n_events), r.integers(0, 2, n_events)
        streams.append((t, (p * 128 * 128 + y * 128 + x).astype(np.int32)))
    ev = _pad(streams)
    layer = ConvLayer(name="conv1", ic=2, h_in=128, w_in=128, oc=32, k=3, s=1, p=0, init_k=1.0,
                      tau=30.0, max_queue_len=n_events + 1, max_out_spikes=8192)
    params = [_params(_codes(w, (32, 2, 3, 3), 24.0, 8), 30.0, 200)]
    return Workload("c4_conv2x32k3_128", Network((2, 128, 128), [layer]), params, ev, "round")


def config5(B=4096, n_events=8192, cap=1 << 21) -> Workload:
    """FC 4096 -> 1024, int16 codes N(0, 512), v_th 64; a quarter of the events share the
    previous event's ms (dt = 0), the other gaps are U{1..4}."""
    w = _weight_rng(5)
    streams = []
    for r in _children(5, B):
        gaps = np.where(r.random(n_events) < 0.25, 0, r.integers(1, 5, n_events))
        gaps[0] = r.integers(0, 5)
        streams.append((np.cumsum(gaps).astype(np.float32),
                        r.integers(0, 4096, n_events).astype(np.int32)))
    layer = FCLayer(name="fc1", n_in=4096, n_out=1024, init_k=1.0, tau=20.0, max_out_spikes=cap)
    params = [_params(_codes(w, (1024, 4096), 512.0, 16), 20.0, 64)]
    return Workload("c5_fc4096x1024", Network((4096,), [layer]), params, _pad(streams), "round")


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}
