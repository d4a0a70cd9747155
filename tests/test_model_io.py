"""Model files (salt_amd.io): network description round trip, float and quantized .npz
files with the reference's keys and JSON sections (salt_core/tests/test_io.py), a file
laid out by hand in that format, and the error cases.  CPU only."""
import json

import numpy as np
import pytest

from salt_amd import ConvLayer, FCLayer, Network, QuantizedLayerParams, RoundMode
from salt_amd.io import (NETWORK_KEY, QUANT_KEY, load_quantized, load_weights,
                         network_from_dict, network_to_dict, save_quantized, save_weights)
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.quant.fixed_point import OverflowMode

# every capacity, chunk_size and dynamics field off its default (test_io.py:17-22)
NETWORK = Network(input_shape=(2, 8, 8), layers=(
    ConvLayer(name="conv1", ic=2, h_in=8, w_in=8, oc=3, k=3, s=2, p=1, init_k=5.0,
              tau=12.0, v_th=0.8, alpha=3.0, chunk_size=4,
              max_queue_len=17, max_out_spikes=40, max_extra_steps=9),
    FCLayer(name="out", n_in=3 * 4 * 4, n_out=5, init_k=2.0, tau=20.0, chunk_size=8)))
METADATA = {"spec": {"bits": 4}, "source": "unit-test", "v_abs_max": [[2.0, 2.0, 2.0], [2.0] * 5]}


def _weights():
    rng = np.random.default_rng(0)
    return [rng.standard_normal(l.weight_shape).astype(np.float32) for l in NETWORK.layers]


def _quant_params():
    rng = np.random.default_rng(1)
    conv = QuantizedLayerParams(
        q=rng.integers(-7, 8, (3, 2, 3, 3)).astype(np.int8),
        decay_table_int=build_decay_table_int(8, 12.0),
        v_th_int=np.full(3 * 4 * 4, 40, np.int32), scale=np.full(3 * 4 * 4, 0.25, np.float32),
        f_a=8, f_V=6, i_V=7, overflow_mode=OverflowMode.WRAP)
    out = QuantizedLayerParams(
        q=rng.integers(-7, 8, (5, 48)).astype(np.int8),
        decay_table_int=build_decay_table_int(8, 20.0), v_th_int=None,
        scale=np.linspace(0.1, 0.5, 5).astype(np.float32), f_a=8, f_V=6, i_V=9,
        overflow_mode="saturate")
    return [conv, out]


def test_dict_roundtrip():
    d = network_to_dict(NETWORK)
    assert d["format"] == 1
    assert [e["type"] for e in d["layers"]] == ["conv", "fc"]
    assert network_from_dict(json.loads(json.dumps(d))) == NETWORK


def test_description_lists_every_layer_field_in_declaration_order():
    d = network_to_dict(NETWORK)
    assert list(d["layers"][0]) == ["type", "name", "ic", "h_in", "w_in", "oc", "k", "s", "p",
                                    "init_k", "tau", "v_th", "alpha", "chunk_size",
                                    "max_queue_len", "max_out_spikes", "max_extra_steps"]
    assert list(d["layers"][1]) == ["type", "name", "n_in", "n_out", "init_k", "tau", "v_th",
                                    "alpha", "chunk_size", "max_out_spikes", "max_extra_steps"]


def test_weights_roundtrip_and_keys(tmp_path):
    w = _weights()
    path = tmp_path / "w.npz"
    save_weights(path, NETWORK, w)
    network, loaded = load_weights(path)
    assert network == NETWORK
    for a, b in zip(w, loaded):
        assert a.dtype == b.dtype and np.array_equal(a, b)
    with np.load(path) as data:
        assert sorted(data.files) == sorted(["conv1", "out", NETWORK_KEY])


def test_unknown_format_and_layer_type_raise():
    d = network_to_dict(NETWORK)
    d["format"] = 2
    with pytest.raises(ValueError, match="format"):
        network_from_dict(d)
    d = network_to_dict(NETWORK)
    d["layers"][1]["type"] = "pool"
    with pytest.raises(ValueError, match="pool"):
        network_from_dict(d)


def test_layer_named_like_network_key_raises(tmp_path):
    net = Network(input_shape=(2, 8, 8), layers=(FCLayer(name=NETWORK_KEY, n_in=128, n_out=5,
                                                         init_k=2.0),))
    with pytest.raises(ValueError, match=NETWORK_KEY):
        save_weights(tmp_path / "w.npz", net, [np.zeros((5, 128), np.float32)])


def test_file_without_network_raises(tmp_path):
    path = tmp_path / "old.npz"
    np.savez(path, out=np.zeros((5, 128), dtype=np.float32))
    with pytest.raises(ValueError, match=NETWORK_KEY):
        load_weights(path)


def test_quantized_roundtrip_every_field_equal(tmp_path):
    params = _quant_params()
    path = tmp_path / "q.npz"
    save_quantized(path, NETWORK, params, "truncate", METADATA)
    model = load_quantized(path)
    assert model.network == NETWORK
    assert model.round_mode is RoundMode.TRUNCATE
    assert model.metadata == METADATA
    for saved, read in zip(params, model.params):
        for f in ("q", "decay_table_int", "scale"):
            a, b = np.asarray(getattr(saved, f)), getattr(read, f)
            assert a.dtype == b.dtype and np.array_equal(a, b)
        assert (read.f_a, read.f_V, read.i_V) == (saved.f_a, saved.f_V, saved.i_V)
        assert read.overflow_mode is OverflowMode(saved.overflow_mode)
    assert np.array_equal(params[0].v_th_int, model.params[0].v_th_int)
    assert model.params[1].v_th_int is None


def test_quantized_npz_keys(tmp_path):
    """salt_core/tests/test_io.py:116-124."""
    path = tmp_path / "q.npz"
    save_quantized(path, NETWORK, _quant_params(), "round", METADATA)
    with np.load(path) as data:
        assert sorted(data.files) == sorted([
            NETWORK_KEY, QUANT_KEY,
            "conv1/q", "conv1/decay_table_int", "conv1/v_th_int", "conv1/scale",
            "out/q", "out/decay_table_int", "out/scale"])
        quant = json.loads(str(data[QUANT_KEY]))
    assert quant == {"format": 1, "round_mode": "round",
                     "layers": {"conv1": {"f_a": 8, "f_V": 6, "i_V": 7, "overflow_mode": "wrap"},
                                "out": {"f_a": 8, "f_V": 6, "i_V": 9, "overflow_mode": "saturate"}},
                     "metadata": METADATA}


def test_loads_a_file_laid_out_by_hand(tmp_path):
    """A model.npz assembled key by key from the published layout (no save_quantized):
    JSON text sections plus per-layer arrays."""
    net_json = ('{"format": 1, "input_shape": [4], "layers": [{"type": "fc", "name": "out", '
                '"n_in": 4, "n_out": 2, "init_k": 1.0, "tau": 4.0, "v_th": 1000000000.0, '
                '"alpha": 2.0, "chunk_size": 1, "max_out_spikes": 16, "max_extra_steps": 0}]}')
    quant_json = ('{"format": 1, "round_mode": "truncate", "layers": {"out": {"f_a": 4, '
                  '"f_V": 1, "i_V": 16, "overflow_mode": "wrap"}}, "metadata": {"decoder": '
                  '"membrane_regression", "batch_size": 8}}')
    path = tmp_path / "model.npz"
    np.savez(path, **{NETWORK_KEY: np.asarray(net_json), QUANT_KEY: np.asarray(quant_json),
                      "out/q": np.array([[50, 1, 2, 3], [45, 0, 0, 0]], np.int16),
                      "out/decay_table_int": np.array([12, 9, 7], np.int32),
                      "out/scale": np.array([1.0, 2.0], np.float32)})
    model = load_quantized(path)
    layer = model.network.layers[0]
    assert (layer.name, layer.n_in, layer.n_out, layer.max_out_spikes) == ("out", 4, 2, 16)
    assert model.round_mode is RoundMode.TRUNCATE
    p = model.params[0]
    assert p.q.dtype == np.int16 and p.q[1, 0] == 45 and p.v_th_int is None
    assert (p.f_a, p.f_V, p.i_V, p.overflow_mode) == (4, 1, 16, OverflowMode.WRAP)
    assert model.metadata == {"decoder": "membrane_regression", "batch_size": 8}


@pytest.mark.parametrize("v_th, where", [
    (np.int32(0), "its scalar threshold"),                           # scalar
    (np.array([40, 40, -3], np.int32), "channel 2"),                 # per channel
    (np.where(np.arange(48) == 21, 0, 40).astype(np.int32), "channel 1 (neuron 21)")])
def test_load_quantized_refuses_nonpositive_thresholds_naming_the_channel(tmp_path, v_th, where):
    """A threshold <= 0 fires on the reference's pad, catch-up and identity columns
    (salt_core/quant/scan.py:46-51), which this path does not run: the model is refused
    when loaded, the message naming the layer and the channel (conv1 has 4 x 4 neurons
    per channel, so neuron 21 is in channel 1)."""
    params = _quant_params()
    params[0] = params[0]._replace(v_th_int=v_th)
    path = tmp_path / "q.npz"
    save_quantized(path, NETWORK, params, "round", METADATA)  # writing stays possible
    with pytest.raises(ValueError, match=rf"conv1: v_th_int = -?\d+ <= 0 at {where.replace('(', '[(]').replace(')', '[)]')}"):
        load_quantized(path)


def test_quantized_param_count_mismatch_raises(tmp_path):
    with pytest.raises(ValueError, match="量化參數"):
        save_quantized(tmp_path / "q.npz", NETWORK, _quant_params()[:1], "round", METADATA)


def test_load_quantized_from_float_weights_file_raises(tmp_path):
    path = tmp_path / "w.npz"
    save_weights(path, NETWORK, _weights())
    with pytest.raises(ValueError, match=QUANT_KEY):
        load_quantized(path)


def test_metadata_must_be_json(tmp_path):
    with pytest.raises(TypeError):
        save_quantized(tmp_path / "q.npz", NETWORK, _quant_params(), "round", {"x": object()})


def test_readout_scales_registers_back_per_neuron():
    """salt_core/tests/test_quant_backend.py:255-273: registers [100, 90], f_V = 1,
    s_c = [1, 2] -> [50, 90]; the argmax moves from neuron 0 to neuron 1."""
    import torch
    from salt_amd.quant_run import readout_scores
    p = QuantizedLayerParams(q=None, decay_table_int=None, v_th_int=None,
                             scale=np.array([1.0, 2.0], np.float32), f_a=4, f_V=1, i_V=16)
    s = readout_scores(torch.tensor([[100, 90]], dtype=torch.int32), p)
    assert s.dtype == np.float32 and s.tolist() == [[50.0, 90.0]]
    assert int(np.argmax([100, 90])) == 0 and int(np.argmax(s[0])) == 1
