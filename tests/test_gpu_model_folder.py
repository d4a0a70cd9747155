"""The quantized-model harness on the GPU: a saved model re-runs bit-exactly,
quant_forward_split's per-sample fields equal the oracle's, over-capacity batches equal
the layer-by-layer path and grow until they fit (run_until_fits), and a model folder
passes --check against reference fields computed by the oracle (and fails it when one
field is changed)."""
import dataclasses
import os

import numpy as np
import pytest
import torch

from helpers import oracle_network, write_nmnist_tree
from salt_amd import ConvLayer, FCLayer, Network, QuantBackend, QuantizedLayerParams
from salt_amd import workloads as W
from salt_amd.capacity import GrowthPolicy
from salt_amd.data import NMNISTDataset, split_input_events
from salt_amd.decoder import MembraneRegressionDecoder
from salt_amd.io import load_quantized, save_quantized
from salt_amd.network import InputEvents
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.quant_run import quant_forward_split, reference_arrays, run_until_fits
from salt_amd.quantize import check, evaluate

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _net(caps=(4096, 4096, 4096), mql=100000, vth=(60, 50)):
    c1 = ConvLayer(name="conv1", ic=2, h_in=34, w_in=34, oc=16, k=5, s=2, p=0, init_k=1.0,
                   tau=10.0, max_queue_len=mql, max_out_spikes=caps[0])
    c2 = ConvLayer(name="conv2", ic=16, h_in=15, w_in=15, oc=32, k=3, s=2, p=0, init_k=1.0,
                   tau=20.0, max_queue_len=mql, max_out_spikes=caps[1])
    out = FCLayer(name="out", n_in=1568, n_out=10, init_k=1.0, tau=40.0, v_th=1e9,
                  max_out_spikes=caps[2])
    rng = np.random.default_rng(42)

    def prm(shape, tau, v, scale, i_V=14):
        q = np.clip(np.round(rng.normal(0, 24, shape)), -127, 127).astype(np.int8)
        return QuantizedLayerParams(q=q, decay_table_int=build_decay_table_int(10, tau),
                                    v_th_int=v, scale=scale, f_a=10, f_V=0, i_V=i_V,
                                    overflow_mode="wrap")
    params = [prm((16, 2, 5, 5), 10.0, np.int32(vth[0]), np.float32(0.5)),
              prm((32, 16, 3, 3), 20.0, np.int32(vth[1]), np.float32(0.25)),
              prm((10, 1568), 40.0, None, rng.uniform(0.5, 2.0, 10).astype(np.float32), i_V=11)]
    return Network((2, 34, 34), [c1, c2, out]), params


def _raw(seed, B, n_mean=300):
    ev = W._pad([W.blob_stream(r, n_mean) for r in
                 [np.random.default_rng(s) for s in np.random.SeedSequence(seed).spawn(B)]])
    return InputEvents(np.asarray(ev.event_times), np.asarray(ev.source_idx),
                       np.asarray(ev.n_real_events))


def _oracle_fields(net, params, raw, rm="round"):
    """The per-sample fields of quant_forward_split from the oracle's layer outputs."""
    refs = oracle_network(net, params, raw, rm)
    last = params[-1]
    scores = (refs[-1]["v_final"].astype(np.float32) * np.float32(2.0 ** -last.f_V)
              * np.asarray(last.scale, np.float32))
    over, trunc = [], []
    for layer, p, r in zip(net.layers, params, refs):
        half = 1 << (p.i_V + p.f_V - 1)
        over.append((r["v_min"] < -half).any(axis=1) | (r["v_max"] > half - 1).any(axis=1))
        t = r["out_n"] > layer.max_out_spikes
        if hasattr(layer, "max_queue_len"):
            t |= r["needed_queue"] > layer.max_queue_len
        trunc.append(t)
    return {"v_final_int": refs[-1]["v_final"],
            "preds": np.argmax(scores, axis=1),
            "spike_count": np.stack([r["out_n"] for r in refs], axis=1),
            "truncated": np.stack(trunc, axis=1),
            "overflowed": np.stack(over, axis=1),
            "v_unfitted_min": np.stack([r["v_min"].min(axis=1) for r in refs], axis=1),
            "v_unfitted_max": np.stack([r["v_max"].max(axis=1) for r in refs], axis=1)}


def test_saved_model_reruns_bit_exact(tmp_path):
    net, params = _net()
    path = tmp_path / "model.npz"
    save_quantized(path, net, params, "truncate", {"decoder": "membrane_regression"})
    model = load_quantized(path)
    raw = _raw(1, 6)
    a = net.apply_batched(params, raw, backend=QuantBackend("truncate"))
    b = model.network.apply_batched(model.params, raw, backend=QuantBackend(model.round_mode))
    for x, y in zip(a.results, b.results):
        assert torch.equal(x.v_final, y.v_final) and torch.equal(x.spike_count, y.spike_count)
        assert torch.equal(x.stream_stats, y.stream_stats)


def test_quant_forward_split_matches_oracle():
    net, params = _net()
    raw = _raw(2, 20)
    print("quant_forward_split 20 samples, batch 7", flush=True)
    out = quant_forward_split(net, MembraneRegressionDecoder(), params, "round", raw, 7, device=DEV)
    want = _oracle_fields(net, params, raw)
    assert 0 < out.overflowed[:, 2].sum() < 20  # the 11-bit FC register overflows in some
    for key, value in want.items():
        np.testing.assert_array_equal(getattr(out, key), value, err_msg=key)
    assert set(out.needed) == {"conv1", "conv2", "out"}
    assert list(out.needed["conv1"]) == ["max_queue_len", "max_out_spikes", "max_extra_steps"]
    np.testing.assert_array_equal(out.needed["conv2"]["max_out_spikes"], want["spike_count"][:, 1])


def test_over_capacity_batches_follow_the_layer_path_and_grow_until_they_fit():
    net, params = _net(caps=(400, 4096, 4096), vth=(30, 50))
    raw = _raw(3, 12)
    print("over capacity: quant_forward_split", flush=True)
    out = quant_forward_split(net, MembraneRegressionDecoder(), params, "round", raw, 5, device=DEV)
    assert out.truncated[:, 0].any()
    # every field equals the layer-by-layer path, which cuts streams as the reference does
    layered = net.apply_batched(params, raw, backend=QuantBackend("round", neuron_extremes=False))
    np.testing.assert_array_equal(out.v_final_int, layered.results[-1].v_final.cpu().numpy())
    for i, r in enumerate(layered.results):
        np.testing.assert_array_equal(out.spike_count[:, i], r.spike_count.cpu().numpy())
        np.testing.assert_array_equal(out.v_unfitted_max[:, i], r.stream_stats[:, 1].cpu().numpy())
    print("over capacity: run_until_fits", flush=True)
    policies = {l.name: GrowthPolicy() for l in net.layers}
    grown, out2, n_regrow = run_until_fits(net, MembraneRegressionDecoder(), params, "round",
                                           raw, 5, policies, device=DEV)
    assert n_regrow >= 1 and not out2.truncated.any()
    assert grown.layers[0].max_out_spikes >= int(out.spike_count[:, 0].max())
    want = _oracle_fields(grown, params, raw)
    for key, value in want.items():
        np.testing.assert_array_equal(getattr(out2, key), value, err_msg=f"grown {key}")


def test_check_and_eval_on_a_model_folder(tmp_path):
    root = str(tmp_path / "N-MNIST")
    write_nmnist_tree(root, per_digit_train=4, per_digit_test=2, seed=9, n_range=(60, 220))
    net, params = _net()
    data_meta = {"max_events": 150, "val_size": 4,
                 "verify": {"split": "val", "seed": 7, "n": 4},
                 "calibration": {"split": "val", "seed": 7, "n": 2}}
    metadata = {"data": data_meta, "decoder": "membrane_regression", "batch_size": 3,
                "growth": {l.name: dataclasses.asdict(GrowthPolicy()) for l in net.layers}}
    folder = tmp_path / "quant"
    folder.mkdir()
    save_quantized(folder / "model.npz", net, params, "round", metadata)
    split = NMNISTDataset(root, max_events=150).build_split(seed=7, n_samples=4, which="val")
    raw = split_input_events(split, net.input_shape)
    want = _oracle_fields(net, params, raw)
    ref = {k: want[k] for k in ("v_final_int", "preds", "spike_count", "truncated", "overflowed")}
    np.savez(folder / "reference.npz", labels=split.labels, **ref)
    print("check: unchanged folder", flush=True)
    assert check(str(folder), root, device=DEV) == 0
    ref["spike_count"] = ref["spike_count"].copy()
    ref["spike_count"][2, 1] += 1
    np.savez(folder / "reference.npz", labels=split.labels, **ref)
    print("check: one field changed", flush=True)
    assert check(str(folder), root, device=DEV) == 1
    print("eval: test pool", flush=True)
    result = evaluate(str(folder), root, "test", None, 0, device=DEV)
    assert result["n_samples"] == 20 and 0.0 <= result["accuracy"] <= 1.0
    assert set(result["headroom_bits"]) == {"conv1", "conv2", "out"}
    assert os.path.exists(folder / "eval" / "test.yaml")
    with np.load(folder / "eval" / "test_outputs.npz") as npz:
        assert npz["preds"].shape == (20,) and npz["labels"].shape == (20,)


def test_overflow_events_match_the_queue_restatement():
    """overflow_events re-runs each overflowing sample in trace mode; every listed event
    (first overflowing step of a neuron) equals the queue restatement's trajectory of that
    layer on the same input stream."""
    from oracle import queue_ref as Q
    from salt_amd.quant_run import MAX_OVERFLOW_EVENTS, overflow_events
    net, params = _net(mql=160)
    raw = _raw(2, 20)
    out = quant_forward_split(net, MembraneRegressionDecoder(), params, "round", raw, 7, device=DEV)
    assert not out.truncated.any() and out.overflowed[:, :2].sum() == 0
    print("overflow_events", flush=True)
    events = overflow_events(net, params, "round", raw, out)
    refs = oracle_network(net, params, raw, "round")
    fc, p = net.layers[2], params[2]
    want = []
    for i in np.nonzero(out.overflowed.any(axis=1))[0]:
        n_in = int(refs[1]["out_n"][i])
        r = Q.fc_forward(p.q, p.decay_table_int, None, p.f_a, p.f_V, p.i_V,
                         refs[1]["out_times"][i], refs[1]["out_src"][i], n_in, 4096,
                         round_mode="round", overflow_mode="wrap")
        for neuron in np.nonzero(r["overflowed"].any(axis=1))[0]:
            step = int(np.argmax(r["overflowed"][neuron]))
            want.append({"sample": int(i), "layer": "out", "channel": int(neuron), "y": 0, "x": 0,
                         "time_ms": float(refs[1]["out_times"][i][step]),
                         "v_before": int(r["v_steps"][neuron, step - 1]) if step > 0 else 0,
                         "v_after": int(r["v_steps"][neuron, step]), "spiked": False,
                         "true_min": int(refs[2]["v_min"][i, neuron]),
                         "true_max": int(refs[2]["v_max"][i, neuron]),
                         "register_range": [-1024, 1023]})
    assert events == want[:MAX_OVERFLOW_EVENTS] and len(events) > 0


def test_converted_params_run_through_the_quantized_network():
    """build_quantized_params output is directly usable (salt_core/tests/
    test_quant_convert.py:96-107): conv 2x2x2 -> FC 8 -> 2, four events."""
    from salt_amd import run_network
    from salt_amd.quant.convert import LayerQuantSpec, build_quantized_params
    from salt_amd.stream import EventStream
    conv = ConvLayer(name="conv", ic=2, h_in=2, w_in=2, oc=2, k=1, s=1, p=0, init_k=5.0,
                     tau=16.0, v_th=1.0, chunk_size=1, max_queue_len=8, max_out_spikes=64)
    fc = FCLayer(name="out", n_in=8, n_out=2, init_k=5.0, tau=16.0, v_th=1e9)
    params = build_quantized_params(
        [conv, fc], (np.array([0.375, 0.125, -1.0, 0.25], np.float32).reshape(2, 2, 1, 1),
                     np.linspace(-0.5, 0.3, 16, dtype=np.float32).reshape(2, 8)),
        [LayerQuantSpec(bits=4, f_a=8, f_V=4), LayerQuantSpec(bits=4, f_a=8, f_V=4, fires=False)],
        [np.array([2.0, 0.5]), np.array([3.0, 1.0])])
    t = torch.arange(1.0, 5.0, device=DEV)
    stream = EventStream(event_times=t, event_source_idx=torch.arange(4, dtype=torch.int32, device=DEV),
                         event_gain=torch.ones(4, device=DEV),
                         n_real_events=torch.tensor(4, dtype=torch.int32, device=DEV))
    out = run_network([conv, fc], params, stream, backend=QuantBackend())
    assert tuple(out.last.v_final.shape) == (2,)
    assert bool(conv.capacity.fits(out.diags[0]))
    # the same run on the CPU oracle
    raw = InputEvents(np.arange(1.0, 5.0, dtype=np.float32)[None], np.arange(4, dtype=np.int32)[None],
                      np.array([4], np.int32))
    refs = oracle_network(Network((2, 2, 2), [conv, fc]), params, raw, "round")
    np.testing.assert_array_equal(out.last.v_final.cpu().numpy(), refs[-1]["v_final"][0])
