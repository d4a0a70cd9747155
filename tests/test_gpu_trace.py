"""Trace mode (salt_layer_trace via layer.forward(..., trace=True)) against the NumPy
queue restatement of salt_core/quant (oracle/queue_ref.py), bit for bit: every neuron's
register after every queue column, the column's spike and overflow flags, and its event
time (NaN past the neuron's real events), for FC and conv layers over thresholds,
overflow and rounding modes, truncated conv queues, padding and stride; plus the
network-level invariants (last column = v_final, spikes per neuron = output stream)."""
import numpy as np
import pytest
import torch

from oracle import queue_ref as Q
from salt_amd import ConvLayer, FCLayer, Network, QuantBackend, QuantizedLayerParams, run_network
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.stream import EventStream, unit_gain
from salt_amd.trace import summarize_trace_scalars

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _stream(rng, B, L, n_src, n_real, t_max=200, pad_time=1e12):
    t = np.full((B, L), pad_time, np.float32)
    s = np.zeros((B, L), np.int32)
    for b in range(B):
        nb = n_real[b]
        t[b, :nb] = np.sort(rng.integers(0, t_max, nb)).astype(np.float32)
        s[b, :nb] = rng.integers(0, n_src, nb)
    return t, s, np.asarray(n_real, np.int32)


def _device(t, s, n):
    tt = torch.from_numpy(t).to(DEV)
    return EventStream(event_times=tt, event_source_idx=torch.from_numpy(s).to(DEV),
                       event_gain=unit_gain(tt), n_real_events=torch.from_numpy(n).to(DEV))


def _params(rng, shape, n, *, f_a, f_V, i_V, mode, vth, tau=8.0, qmax=60):
    q = rng.integers(-qmax, qmax + 1, shape).astype(np.int16)
    return QuantizedLayerParams(q=q, decay_table_int=build_decay_table_int(f_a, tau),
                                v_th_int=vth, scale=np.float32(1.0), f_a=f_a, f_V=f_V,
                                i_V=i_V, overflow_mode=mode)


def _vth_np(p, n):
    if p.v_th_int is None:
        return None
    return np.broadcast_to(np.asarray(p.v_th_int).astype(np.int32), (n,))


def _compare(tr, b, ref, ms, tag):
    np.testing.assert_array_equal(tr.v_steps[b].cpu().numpy(), ref["v_steps"], err_msg=f"{tag} v_steps")
    np.testing.assert_array_equal(tr.spike_mask[b].cpu().numpy(), ref["spike_mask"], err_msg=f"{tag} spikes")
    np.testing.assert_array_equal(tr.overflowed[b].cpu().numpy(), ref["overflowed"], err_msg=f"{tag} overflow")
    np.testing.assert_array_equal(tr.event_ms[b].cpu().numpy(), ms, err_msg=f"{tag} event_ms")


FC_CASES = [
    # (name, f_a, f_V, i_V, overflow, round, vth kind)
    ("scalar_wrap_round", 6, 2, 10, "wrap", "round", "scalar"),
    ("per_neuron_saturate_truncate", 4, 0, 8, "saturate", "truncate", "per_neuron"),
    ("silent_wrap", 10, 0, 9, "wrap", "round", "none"),
]


@pytest.mark.parametrize("case", FC_CASES, ids=[c[0] for c in FC_CASES])
def test_fc_trace_matches_queue_restatement(case):
    name, f_a, f_V, i_V, mode, rm, kind = case
    rng = np.random.default_rng(len(name))
    n_in, n_out, B, L = 40, 24, 3, 150
    vth = {"scalar": np.int32(90 << f_V), "none": None,
           "per_neuron": rng.integers(20, 120, n_out).astype(np.int32)}[kind]
    layer = FCLayer(name="fc", n_in=n_in, n_out=n_out, init_k=1.0, max_out_spikes=4096)
    p = _params(rng, (n_out, n_in), n_out, f_a=f_a, f_V=f_V, i_V=i_V, mode=mode, vth=vth)
    t, s, n = _stream(rng, B, L, n_in, [150, 97, 0])
    print("fc trace", name, flush=True)
    out = layer.forward(p, _device(t, s, n), backend=QuantBackend(rm), trace=True)
    torch.cuda.synchronize()
    tr = out.trace
    assert tr.v_steps.shape == (B, n_out, L)
    for b in range(B):
        ref = Q.fc_forward(p.q, p.decay_table_int, _vth_np(p, n_out), f_a, f_V, i_V, t[b], s[b],
                           n[b], 4096, round_mode=rm, overflow_mode=mode)
        ms = np.where(np.arange(L) < n[b], t[b], np.nan).astype(np.float32)
        _compare(tr, b, ref, np.broadcast_to(ms, (n_out, L)), f"{name} b={b}")
        np.testing.assert_array_equal(tr.v_steps[b, :, -1].cpu().numpy(),
                                      out.result.v_final[b].cpu().numpy())
    if mode == "wrap" and i_V + f_V <= 10:
        assert bool(tr.overflowed.any())


CONV_CASES = [
    # (name, ic, h, w, oc, k, s, p, mql, f_a, f_V, i_V, overflow, round, vth kind)
    ("k3s1p0_catchup", 2, 10, 10, 3, 3, 1, 0, 40, 6, 0, 12, "wrap", "round", "scalar"),
    ("k3s2p1_truncated_queue", 2, 12, 12, 4, 3, 2, 1, 3, 5, 1, 10, "wrap", "truncate", "per_channel"),
    ("k5s2p2_saturate_per_neuron", 1, 11, 11, 2, 5, 2, 2, 30, 4, 0, 8, "saturate", "round", "per_neuron"),
    ("k2s2p0_silent", 3, 8, 8, 2, 2, 2, 0, 12, 8, 2, 9, "wrap", "round", "none"),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv_trace_matches_queue_restatement(case):
    name, ic, h, w, oc, k, st, pd, mql, f_a, f_V, i_V, mode, rm, kind = case
    rng = np.random.default_rng(100 + len(name))
    layer = ConvLayer(name="conv", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=st, p=pd, init_k=1.0,
                      max_queue_len=mql, max_out_spikes=8192)
    nn, hw = layer.n_neurons, layer.h_out * layer.w_out
    vth = {"scalar": np.int32(70), "none": None,
           "per_channel": np.repeat(rng.integers(20, 90, oc), hw).astype(np.int32),
           "per_neuron": rng.integers(10, 60, nn).astype(np.int32)}[kind]
    p = _params(rng, (oc, ic, k, k), nn, f_a=f_a, f_V=f_V, i_V=i_V, mode=mode, vth=vth)
    B, L = 3, 260
    t, s, n = _stream(rng, B, L, ic * h * w, [260, 120, 1])
    print("conv trace", name, flush=True)
    out = layer.forward(p, _device(t, s, n), backend=QuantBackend(rm), trace=True)
    torch.cuda.synchronize()
    tr = out.trace
    assert tr.v_steps.shape == (B, nn, mql)
    truncated = False
    for b in range(B):
        ref = Q.conv_forward(p.q, p.decay_table_int, _vth_np(p, nn), f_a, f_V, i_V, t[b], s[b],
                             n[b], 8192, ic=ic, h_in=h, w_in=w, k=k, s=st, p=pd,
                             max_queue_len=mql, round_mode=rm, overflow_mode=mode)
        x, y, c = Q.unravel_conv_source(s[b], h, w)
        sc = Q.build_conv_structure(t[b], x, y, c, k, st, pd, layer.h_out, layer.w_out, mql, n[b])
        l2g = np.minimum(sc["local_to_global_j"], L - 1)
        idle = np.arange(mql)[None, :] >= sc["n_real_events"][:, None]
        ms = np.where(idle, np.nan, t[b][l2g]).astype(np.float32)
        truncated |= bool((sc["n_real_events"] > mql).any())
        _compare(tr, b, ref, Q.tile_channels(ms, oc), f"{name} b={b}")
        np.testing.assert_array_equal(tr.v_steps[b, :, -1].cpu().numpy(),
                                      out.result.v_final[b].cpu().numpy())
    if mql < 5:
        assert truncated


def test_network_trace_invariants():
    rng = np.random.default_rng(7)
    c1 = ConvLayer(name="conv1", ic=2, h_in=10, w_in=10, oc=3, k=3, s=1, p=1, init_k=1.0,
                   max_queue_len=64, max_out_spikes=2048)
    out = FCLayer(name="out", n_in=300, n_out=6, init_k=1.0, max_out_spikes=2048)
    net = Network((2, 10, 10), [c1, out])
    params = [_params(rng, (3, 2, 3, 3), 300, f_a=6, f_V=0, i_V=12, mode="wrap", vth=np.int32(50)),
              _params(rng, (6, 300), 6, f_a=6, f_V=0, i_V=12, mode="wrap", vth=None)]
    t, s, n = _stream(rng, 2, 180, 200, [180, 150])
    res = run_network(net.layers, params, _device(t, s, n), backend=QuantBackend("round"),
                      trace=True)
    torch.cuda.synchronize()
    assert len(res.traces) == 2
    for r, tr in zip(res.results, res.traces):
        assert torch.equal(tr.v_steps[:, :, -1], r.v_final)
        assert torch.equal(tr.spike_mask.sum(dim=(1, 2)).to(torch.int32), r.spike_count)
    summary = summarize_trace_scalars(type(res.traces[0])(*(x[0] for x in res.traces[0])))
    assert summary["n"] == 300 and summary["steps"] == 64
    assert summary["total_spikes"] == int(res.results[0].spike_count[0])
    assert 0.0 < summary["idle_frac"] < 1.0 and summary["nonfinite_v"] == 0
