"""Host-side API (no GPU): input checks, network wiring, parameter validation, layer
geometry -- mirroring salt_core/tests/test_network.py, test_layer_connections.py and the
ValueErrors of salt_core/quant."""
import numpy as np
import pytest

from salt_amd import (ConvLayer, FCLayer, InputEvents, Network, QuantizedLayerParams, conv, fc)
from salt_amd.quant.backend import prepare_params, reference_truncation
from salt_amd.quant.codes import build_decay_table_int


def _raw(times, n_real):
    return (np.array(times, dtype=np.float32), np.zeros(len(times), dtype=np.int32), np.array(n_real))


def test_checked_accepts_valid_times_and_ignores_pad():
    """salt_core/tests/test_network.py:22-25."""
    assert isinstance(InputEvents.checked(*_raw([0.0, 3.0, 3.0, 1e12], n_real=3)), InputEvents)


@pytest.mark.parametrize("times, message", [
    ([1.0, 2.5, 4.0], "整數"),
    ([-1.0, 2.0, 4.0], r"\[0, 2\^31\)"),
    ([1.0, 2.0, 2.0 ** 31], r"\[0, 2\^31\)"),
    ([1.0, 5.0, 4.0], "不遞減"),
])
def test_checked_rejects_invalid_real_times(times, message):
    """salt_core/tests/test_network.py:28-36."""
    with pytest.raises(ValueError, match=message):
        InputEvents.checked(np.array(times, dtype=np.float64), np.zeros(3, np.int32), np.array(3))


def test_checked_rejects_times_that_round_to_2_31_in_float32():
    """A float64 time just below 2^31 passes the reference's check but is 2^31 once cast to
    the float32 the kernels read; it is rejected here with the range message.  The largest
    float32 below 2^31 (2^31 - 128) is accepted."""
    with pytest.raises(ValueError, match=r"\[0, 2\^31\)"):
        InputEvents.checked(np.array([1.0, 2.0 ** 31 - 10]), np.zeros(2, np.int32), np.array(2))
    InputEvents.checked(np.array([1.0, 2.0 ** 31 - 128]), np.zeros(2, np.int32), np.array(2))


def test_checked_accepts_batch():
    """salt_core/tests/test_network.py:39-42."""
    InputEvents.checked(np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 0.0]]), np.zeros((2, 3), np.int32),
                        np.array([3, 2]))


def test_network_build_names_and_shapes():
    net = Network.build((2, 34, 34), [conv(16, k=5, s=2, p=0, init_k=1.0),
                                      conv(32, k=3, s=2, p=0, init_k=1.0), fc(10, init_k=1.0)])
    assert [l.name for l in net.layers] == ["conv1", "conv2", "fc1"]
    assert net.layers[0].output_shape == (16, 15, 15)
    assert net.layers[1].output_shape == (32, 7, 7)
    assert net.layers[2].n_in == 32 * 7 * 7


def test_network_rejects_unconnected_layers():
    with pytest.raises(ValueError):
        Network((2, 8, 8), [FCLayer(name="a", n_in=128, n_out=4, init_k=1.0),
                            ConvLayer(name="b", ic=1, h_in=2, w_in=2, oc=1, k=1, s=1, p=0, init_k=1.0)])


def test_conv_geometry_and_capacity():
    layer = ConvLayer(name="c", ic=2, h_in=34, w_in=34, oc=16, k=5, s=2, p=0, init_k=1.0)
    assert (layer.h_out, layer.w_out, layer.n_neurons) == (15, 15, 3600)
    assert dict(layer.capacity) == {"max_queue_len": 128, "max_out_spikes": 8192, "max_extra_steps": 0}
    with pytest.raises(ValueError):
        ConvLayer(name="bad", ic=1, h_in=2, w_in=2, oc=1, k=5, s=1, p=0, init_k=1.0)
    v = np.arange(layer.n_neurons)
    assert layer.unflatten_neurons(v).shape == (16, 15, 15)
    assert layer.broadcast_channels(np.arange(16)).shape == (3600,)


def _fc_params(**kw):
    base = dict(q=np.array([[5, 3], [2, 1]]), decay_table_int=build_decay_table_int(4, 4.0),
                v_th_int=np.array([8, 8]), scale=np.float32(1.0), f_a=4, f_V=0, i_V=16)
    base.update(kw)
    return QuantizedLayerParams(**base)


FC = FCLayer(name="out", n_in=2, n_out=2, init_k=5.0, tau=4.0)


@pytest.mark.parametrize("kw, match", [
    (dict(q=np.array([[0.01, -0.02], [0.03, 0.0]])), "整數"),   # quant/backend.py:14-20
    (dict(f_a=16), "MAX_SHIFT_BITS"),                          # fixed_point.py:57-60
    (dict(i_V=29, f_V=2), "MAX_REGISTER_BITS"),                # fixed_point.py:79-82
    (dict(overflow_mode="clip"), "clip"),                      # fixed_point.py:78
    (dict(v_th_int=np.array([0, 8])), "v_th_int <= 0"),        # rejected on purpose
    (dict(decay_table_int=np.zeros(0, np.int32)), "empty"),
    (dict(decay_table_int=np.array([16, 3])), r"\[0, 2\^f_a\)"),
    (dict(q=np.zeros((3, 2), np.int32)), "shape"),
])
def test_params_validation_errors(kw, match):
    with pytest.raises(ValueError, match=match):
        prepare_params(FC, _fc_params(**kw), device=None)


def test_reference_truncation_keeps_neuron_major_prefix():
    """salt_core/stream.py:49-64: nonzero(size=cap) is neuron-major, then a stable sort by
    event.  Spikes (event j, neuron): (0,2) (1,0) (1,2) (2,1) (3,0); cap 3 keeps neuron 0's
    two spikes and neuron 1's one -> (1,0) (2,1) (3,0)."""
    times = np.array([[0, 1, 1, 2, 3]], np.float32)
    src = np.array([[2, 0, 2, 1, 0]], np.int32)
    t, s = reference_truncation(times, src, np.array([5]), 3, 3)
    assert s[0].tolist() == [0, 1, 0] and t[0].tolist() == [1.0, 2.0, 3.0]
    t, s = reference_truncation(times, src, np.array([5]), 6, 3)
    assert s[0].tolist() == [2, 0, 2, 1, 0, 0] and t[0, 5] == np.float32(1e12)


def test_weight_codes_wrap_to_int32_and_int32_tables_are_not_copied():
    """q → int32 with two's-complement wrap, as jnp.asarray(q, jnp.int32) gives
    (salt_core/quant/backend.py:14-20 takes the codes as int32); an int32 table is used as
    it is, and its narrowest code width is chosen from its range."""
    from salt_amd.quant.backend import _as_int32, _code_bits
    q64 = np.array([2 ** 31, -2 ** 31 - 1, 2 ** 32 + 5, -7, 127], np.int64)
    np.testing.assert_array_equal(_as_int32(q64), np.array([-2 ** 31, 2 ** 31 - 1, 5, -7, 127]))
    assert _as_int32(q64).dtype == np.int32
    qu = np.array([255, 128, 0], np.uint8)
    np.testing.assert_array_equal(_as_int32(qu), [255, 128, 0])
    q32 = np.arange(-5, 5, dtype=np.int32).reshape(2, 5)
    assert _as_int32(q32) is q32
    codes, bits = _code_bits(q32)
    assert bits == 8 and codes.dtype == np.int8
    np.testing.assert_array_equal(codes, q32)
    wide = np.array([[70000, -3]], np.int32)
    codes, bits = _code_bits(wide)
    assert bits == 32 and np.shares_memory(codes, wide)
    codes, bits = _code_bits(np.array([[-32768, 32767]], np.int32))
    assert bits == 16 and codes.dtype == np.int16
