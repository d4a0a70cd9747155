"""The five benchmark configurations on the GPU against the CPU oracle, layer by layer:
spike streams, final registers, per-neuron extremes and needed capacities bit for bit.
Config 5 (about 1.5 M spikes per stream) is compared at its full batch through per-stream
order-sensitive hashes, counts, final registers and extremes of every stream, plus entry by
entry on sampled streams."""
import numpy as np
import pytest
import torch

from salt_amd import QuantBackend
from salt_amd import workloads as W
from salt_amd.stream import stream_hash
from oracle import oracle as O
from helpers import assert_layer_equal, oracle_spec

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cid", [1, 2, 3, 4])
def test_config_layers_match_oracle(cid):
    w = W.CONFIGS[cid]()
    print("config", cid, w.name, w.events.event_times.shape, flush=True)
    backend = QuantBackend(round_mode=w.round_mode, neuron_extremes=True)
    stream = w.network.input_stream(w.events)
    t, s, n = w.events
    for layer, params in zip(w.network.layers, w.params):
        out = layer.forward(params, stream, backend=backend)
        torch.cuda.synchronize()
        geom, prm, cap = oracle_spec(layer, params, w.round_mode)
        ref = O.layer_forward(geom, prm, t, s, n, cap)
        assert_layer_equal(out, ref, tag=f"config{cid}/{layer.name}")
        assert bool(layer.capacity.fits(out.diag).all()), f"{layer.name} capacity"
        stream = out.stream
        t, s, n = ref["out_times"], ref["out_src"], ref["out_n"]


@pytest.mark.timeout(900)
def test_config5_every_stream_at_full_batch():
    """Configuration 5 at its benchmark batch (4096 streams of 8192 events, ~1.5 M spikes
    per stream): every stream's spike count, order-sensitive hash, final registers and
    extremes against the oracle's hash mode, and 12 sampled streams entry by entry."""
    w = W.config5()
    B = w.events.event_times.shape[0]
    assert B == 4096
    layer, params = w.network.layers[0], w.params[0]
    backend = QuantBackend(round_mode=w.round_mode, neuron_extremes=False)
    print("config5: GPU forward", flush=True)
    out = layer.forward(params, w.network.input_stream(w.events), backend=backend)
    hashes = stream_hash(out.stream).cpu().numpy().view(np.uint64)
    counts = out.stream.n_real_events.cpu().numpy()
    v_final = out.result.v_final.cpu().numpy()
    st = out.result.stream_stats.cpu().numpy()
    cap = layer.max_out_spikes
    sample = np.random.default_rng(0).choice(B, 12, replace=False)
    got_t = out.stream.event_times[torch.as_tensor(sample, device=out.stream.event_times.device)].cpu().numpy()
    got_s = out.stream.event_source_idx[torch.as_tensor(sample, device=out.stream.event_times.device)].cpu().numpy()
    del out
    torch.cuda.empty_cache()
    geom, prm, cap = oracle_spec(layer, params, w.round_mode)
    t, s, n = w.events
    step = 512
    for b0 in range(0, B, step):
        sl = slice(b0, b0 + step)
        ref = O.layer_forward(geom, prm, t[sl], s[sl], n[sl], cap, hashed=True)
        np.testing.assert_array_equal(counts[sl], ref["out_n"], err_msg=f"counts {b0}")
        bad = np.nonzero(hashes[sl] != ref["out_hash"])[0]
        assert bad.size == 0, f"stream hashes differ from the oracle at streams {b0 + bad[:8]}"
        np.testing.assert_array_equal(v_final[sl], ref["v_final"], err_msg=f"v_final {b0}")
        np.testing.assert_array_equal(st[sl, 0], ref["v_min"].min(axis=1), err_msg=f"vmin {b0}")
        np.testing.assert_array_equal(st[sl, 1], ref["v_max"].max(axis=1), err_msg=f"vmax {b0}")
        print(f"config5: streams {b0}..{b0 + step - 1} equal", flush=True)
    ref = O.layer_forward(geom, prm, t[sample], s[sample], n[sample], cap)
    for i, b in enumerate(sample):
        m = min(int(counts[b]), cap)
        np.testing.assert_array_equal(got_t[i, :m], ref["out_times"][i, :m], err_msg=f"times {b}")
        np.testing.assert_array_equal(got_s[i, :m], ref["out_src"][i, :m], err_msg=f"src {b}")
    assert counts.min() > 1_000_000  # the high-fire regime is exercised
