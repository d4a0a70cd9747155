"""The reference's known-answer vectors through the GPU path (libsalt_hip.so)."""
import numpy as np
import pytest

from salt_amd import ConvLayer, FCLayer, Network, QuantBackend, QuantizedLayerParams, InputEvents
from salt_amd.quant.codes import build_decay_table_int
from gpu_util import run_layer

pytestmark = pytest.mark.gpu


def _layer_and_params(c):
    if c["kind"] == "fc":
        layer = FCLayer(name="fc", n_in=c["n_in"], n_out=c["n_out"], init_k=1.0, tau=c["tau"],
                        max_out_spikes=c["max_out_spikes"])
    else:
        layer = ConvLayer(name="conv", ic=c["ic"], h_in=c["h_in"], w_in=c["w_in"], oc=c["oc"],
                          k=c["k"], s=c["s"], p=c["p"], init_k=1.0, tau=c["tau"],
                          max_queue_len=c["max_queue_len"], max_out_spikes=c["max_out_spikes"])
    params = QuantizedLayerParams(q=np.array(c["q"]), decay_table_int=build_decay_table_int(c["f_a"], c["tau"]),
                                  v_th_int=None if c["v_th"] is None else np.array(c["v_th"]),
                                  scale=np.float32(1.0), f_a=c["f_a"], f_V=c["f_V"], i_V=c["i_V"],
                                  overflow_mode=c.get("overflow", "wrap"))
    return layer, params


@pytest.mark.parametrize("section", ["layers", "stream_order"])
def test_layer_literals_on_gpu(golden, section):
    for c in golden[section]:
        print("case:", c["cite"], flush=True)
        layer, params = _layer_and_params(c)
        out = run_layer(layer, params, np.array([c["times"]]), np.array([c["src"]]),
                        np.array([c["n_real"]]))
        if "want_v_final" in c:
            assert out.result.v_final[0].tolist() == c["want_v_final"], c["cite"]
        if "want_n" in c:
            assert int(out.stream.n_real_events[0]) == c["want_n"], c["cite"]
        if "want_out_src" in c:
            n = len(c["want_out_src"])
            assert out.stream.event_source_idx[0, :n].tolist() == c["want_out_src"], c["cite"]
        if "want_out_times" in c:
            n = len(c["want_out_times"])
            assert out.stream.event_times[0, :n].tolist() == c["want_out_times"], c["cite"]
        if "want_needed_queue" in c:
            assert int(out.diag.needed["max_queue_len"][0]) == c["want_needed_queue"], c["cite"]
            assert bool(layer.capacity.fits(out.diag)[0]) == (c["want_needed_queue"] <= layer.max_queue_len)


def test_readout_multiplies_back_per_neuron_scale():
    """salt_core/tests/test_quant_backend.py:257-273: registers [100, 90], f_V=1,
    s_c=[1, 2] -> [50, 90]; argmax flips after readout."""
    layer = FCLayer(name="out", n_in=1, n_out=2, init_k=5.0, tau=4.0, max_out_spikes=4)
    params = QuantizedLayerParams(q=np.array([[50], [45]]), decay_table_int=build_decay_table_int(4, 4.0),
                                  v_th_int=None, scale=np.array([1.0, 2.0], np.float32), f_a=4,
                                  f_V=1, i_V=16)
    out = run_layer(layer, params, np.array([[0.0]]), np.array([[0]]), np.array([1]))
    assert out.result.v_final[0].tolist() == [100, 90]
    ro = QuantBackend().readout(out.result, params)
    assert np.allclose(ro.v_final[0].cpu().numpy(), [50.0, 90.0])
    assert int(out.result.v_final[0].argmax()) == 0 and int(ro.v_final[0].argmax()) == 1


def test_network_chains_conv_into_fc_like_manual_chaining():
    """salt_core/tests/test_quant_backend.py:160-183: run_network equals calling the layers
    one by one and feeding each output stream to the next."""
    conv = ConvLayer(name="conv", ic=1, h_in=3, w_in=3, oc=1, k=3, s=1, p=0, init_k=5.0, tau=4.0,
                     max_queue_len=10, max_out_spikes=9)
    fcl = FCLayer(name="out", n_in=1, n_out=2, init_k=5.0, tau=4.0)
    rng = np.random.default_rng(0)
    params = [QuantizedLayerParams(q=rng.integers(-20, 21, (1, 1, 3, 3)), decay_table_int=build_decay_table_int(8, 4.0),
                                   v_th_int=np.array([30]), scale=np.float32(1), f_a=8, f_V=2, i_V=16),
              QuantizedLayerParams(q=rng.integers(-20, 21, (2, 1)), decay_table_int=build_decay_table_int(8, 4.0),
                                   v_th_int=np.array([1000, 1000]), scale=np.float32(1), f_a=8, f_V=2, i_V=16)]
    net = Network((1, 3, 3), [conv, fcl])
    raw = InputEvents(np.arange(1.0, 10.0, dtype=np.float32), np.arange(9, dtype=np.int32), np.array(9))
    out = net.apply(params, raw)
    mid = conv.forward(params[0], net.input_stream(raw))
    want = fcl.forward(params[1], mid.stream)
    assert out.last.v_final.tolist() == want.result.v_final.tolist()
    assert len(out.diags) == 2 and bool(out.fits)
