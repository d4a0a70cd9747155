"""A whole network in one salt_network_forward call (NetworkRunner.run) against the CPU
oracle, bit for bit: every layer's spike stream, final registers and per-stream
statistics, over overflow modes, f_V, threshold kinds, firing FC outputs and truncated
conv queues; and against one salt_layer_forward call per layer (run_layers), with and
without per-neuron extremes and when a stream exceeds an output capacity."""
import zlib

import numpy as np
import pytest
import torch

from salt_amd import ConvLayer, FCLayer, Network, QuantizedLayerParams
from salt_amd import workloads as W
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.runner import NetworkRunner
from helpers import oracle_network

pytestmark = pytest.mark.gpu


def _net(rng, *, f_a, f_V, i_V, overflow, vth, fc_vth, mql1=None, caps=(32768, 32768, 65536),
         taus=(10.0, 20.0, 40.0)):
    c1 = ConvLayer(name="conv1", ic=2, h_in=34, w_in=34, oc=16, k=5, s=2, p=0, init_k=1.0,
                   tau=taus[0], max_queue_len=mql1 or 100000, max_out_spikes=caps[0])
    c2 = ConvLayer(name="conv2", ic=16, h_in=15, w_in=15, oc=32, k=3, s=2, p=0, init_k=1.0,
                   tau=taus[1], max_queue_len=100000, max_out_spikes=caps[1])
    out = FCLayer(name="out", n_in=32 * 7 * 7, n_out=10, init_k=1.0, tau=taus[2],
                  max_out_spikes=caps[2])

    def prm(shape, tau, v):
        q = np.clip(np.round(rng.normal(0, 24, shape)), -127, 127).astype(np.int8)
        return QuantizedLayerParams(q=q, decay_table_int=build_decay_table_int(f_a, tau),
                                    v_th_int=v, scale=np.float32(1.0), f_a=f_a, f_V=f_V,
                                    i_V=i_V, overflow_mode=overflow)
    params = [prm((16, 2, 5, 5), taus[0], vth(16, 15 * 15)),
              prm((32, 16, 3, 3), taus[1], vth(32, 7 * 7)),
              prm((10, 1568), taus[2], fc_vth)]
    return Network((2, 34, 34), [c1, c2, out]), params


def _events(seed, B=24, n_mean=600):
    streams = [W.blob_stream(r, n_mean) for r in
               [np.random.default_rng(s) for s in np.random.SeedSequence(seed).spawn(B)]]
    return W._pad(streams)


def _device_stream(net, ev):
    return net.input_stream(ev, device=torch.device("cuda", 0))


def _compare(outs, refs, tag):
    for i, (o, r) in enumerate(zip(outs, refs)):
        n = o.n.cpu().numpy()
        np.testing.assert_array_equal(n, r["out_n"], err_msg=f"{tag} layer {i} counts")
        cap = r["out_src"].shape[1]
        real = np.arange(cap)[None, :] < np.minimum(r["out_n"], cap)[:, None]
        for got, want, what in ((o.src.cpu().numpy(), r["out_src"], "sources"),
                                (o.times.cpu().numpy(), r["out_times"], "times")):
            np.testing.assert_array_equal(np.where(real, got, 0), np.where(real, want, 0),
                                          err_msg=f"{tag} layer {i} spike {what}")
        np.testing.assert_array_equal(o.v_final.cpu().numpy(), r["v_final"],
                                      err_msg=f"{tag} layer {i} v_final")
        st = o.stats.cpu().numpy()
        np.testing.assert_array_equal(st[:, 0], r["v_min"].min(axis=1), err_msg=f"{tag} layer {i} vmin")
        np.testing.assert_array_equal(st[:, 1], r["v_max"].max(axis=1), err_msg=f"{tag} layer {i} vmax")
        if "needed_queue" in r:
            np.testing.assert_array_equal(st[:, 2], r["needed_queue"], err_msg=f"{tag} layer {i} needed")


def _scalar(v):
    return lambda oc, hw: np.int32(v)


def _per_channel(rng, lo, hi):
    return lambda oc, hw: np.repeat(rng.integers(lo, hi, oc), hw).astype(np.int32)


CASES = [
    # (name, f_a, f_V, i_V, overflow, round)
    ("c3_defaults", 10, 0, 24, "wrap", "round"),
    ("saturate_truncate", 6, 0, 12, "saturate", "truncate"),
    ("wide_codes_fV3", 8, 3, 16, "wrap", "round"),
    ("narrow_wrap_overflow", 4, 2, 10, "wrap", "truncate"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_network_matches_oracle(case):
    name, f_a, f_V, i_V, overflow, rm = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    hi = max(2, min(2 ** (i_V + f_V - 1) - 1, 200 << f_V))
    net, params = _net(rng, f_a=f_a, f_V=f_V, i_V=i_V, overflow=overflow,
                       vth=_per_channel(rng, 1, hi) if f_V else _scalar(min(128, hi)),
                       fc_vth=np.int32(max(1, hi // 2)))
    ev = _events(7 + f_a)
    print("network case", name, flush=True)
    runner = NetworkRunner(net, params, rm)
    outs = runner.run(_device_stream(net, ev))
    torch.cuda.synchronize()
    refs = oracle_network(net, params, ev, rm)
    assert all(int(r["out_n"].max()) <= l.max_out_spikes for r, l in zip(refs, net.layers))
    _compare(outs, refs, name)


def test_network_with_truncated_queues_and_silent_readout():
    """Small max_queue_len on conv1 (events dropped, no catch-up column) and an FC with
    v_th = None, as in the benchmark network."""
    rng = np.random.default_rng(3)
    net, params = _net(rng, f_a=10, f_V=0, i_V=24, overflow="wrap", vth=_scalar(128),
                       fc_vth=None, mql1=12)
    ev = _events(11, B=16, n_mean=900)
    runner = NetworkRunner(net, params, "round")
    outs = runner.run(_device_stream(net, ev))
    torch.cuda.synchronize()
    refs = oracle_network(net, params, ev, "round")
    assert int(refs[0]["needed_queue"].max()) > 12  # truncation happened
    _compare(outs, refs, "truncated queues")


def _same(a, b, tag):
    for i, (x, y) in enumerate(zip(a, b)):
        assert bool((x.n == y.n).all()), f"{tag} layer {i} counts"
        cap = x.src.shape[1]
        real = torch.arange(cap, device=x.n.device)[None, :] < x.n.clamp(max=cap)[:, None]
        for u, v, what in ((x.src, y.src, "sources"), (x.times, y.times, "times")):
            assert bool(((u == v) | ~real).all()), f"{tag} layer {i} {what}"
        for f in ("v_final", "stats", "v_min", "v_max"):
            u, v = getattr(x, f), getattr(y, f)
            assert (u is None) == (v is None), f"{tag} layer {i} {f}"
            if u is not None:
                assert bool((u == v).all()), f"{tag} layer {i} {f}"


@pytest.mark.parametrize("extremes", [False, True])
def test_network_call_matches_layer_calls_on_benchmark_streams(extremes):
    w = W.config3(B=64, n_mean=4500)
    stream = _device_stream(w.network, w.events)
    runner = NetworkRunner(w.network, w.params, w.round_mode)
    one = runner.run(stream, extremes=extremes)
    per_layer = runner.run_layers(stream, extremes=extremes)
    torch.cuda.synchronize()
    _same(one, per_layer, f"extremes={extremes}")
    # the last layer's stream is padded as the reference's is
    last = one[-1]
    cap = last.times.shape[1]
    pad = torch.arange(cap, device=last.n.device)[None, :] >= last.n.clamp(max=cap)[:, None]
    assert bool((last.times[pad] == 1e12).all()) and bool((last.src[pad] == 0).all())


def test_network_over_capacity_feeds_the_capped_stream():
    """A stream whose conv1 spikes exceed max_out_spikes: the next layer reads the first
    cap spikes of it, the same in one call as layer by layer, and fits is false."""
    rng = np.random.default_rng(5)
    net, params = _net(rng, f_a=10, f_V=0, i_V=24, overflow="wrap", vth=_scalar(40),
                       fc_vth=None, caps=(64, 8192, 8192))
    ev = _events(13, B=8, n_mean=800)
    runner = NetworkRunner(net, params, "round")
    stream = _device_stream(net, ev)
    one = runner.run(stream)
    per_layer = runner.run_layers(stream)
    torch.cuda.synchronize()
    assert int(one[0].n.max()) > 64
    _same(one, per_layer, "over capacity")
    assert not runner.check_fits(one).all()


@pytest.mark.parametrize("caps, overflows", [((64, 8192, 8192), True), ((32768, 32768, 65536), False)])
def test_run_network_checks_capacities_once_and_redoes_an_overflowing_layer(caps, overflows):
    """run_network (behind Network.apply_batched) enqueues every layer without a host
    synchronisation and checks the spike counts once at the end; when a stream overflowed
    a layer's capacity, that layer and every later one are run again with the reference's
    truncation.  Either way the result equals chaining layer.forward, which truncates
    each layer exactly before the next reads it."""
    from salt_amd.network import run_network
    from salt_amd.quant.backend import QuantBackend
    rng = np.random.default_rng(9)
    net, params = _net(rng, f_a=10, f_V=0, i_V=24, overflow="wrap", vth=_scalar(40),
                       fc_vth=np.int32(60), caps=caps)
    stream = _device_stream(net, _events(17, B=8, n_mean=800))
    be = QuantBackend("round")
    got = run_network(net.layers, params, stream, backend=be)
    want, s = [], stream
    for layer, p in zip(net.layers, params):
        out = layer.forward(p, s, backend=be)
        want.append(out)
        s = out.stream
    counts = [o.diag.spike_count for o in want]
    assert bool((counts[0] > caps[0]).any()) == overflows
    for i, (r, o) in enumerate(zip(got.results, want)):
        assert bool((r.spike_count == o.result.spike_count).all()), f"layer {i} counts"
        for f in ("v_final", "v_unfitted_min", "v_unfitted_max", "stream_stats"):
            assert bool((getattr(r, f) == getattr(o.result, f)).all()), f"layer {i} {f}"
    assert bool(got.fits.all()) == (not overflows)
