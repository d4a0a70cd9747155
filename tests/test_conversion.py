"""Offline conversion (salt_amd.quant.codes / ptq / convert, salt_amd.fpga_export) against
the hand-computed literals of salt_core/tests/test_quant_codes.py, test_quant_convert.py
and test_fpga_export.py, plus closed-form properties.  CPU only."""
import numpy as np
import pytest

from salt_amd import ConvLayer, FCLayer, QuantizedLayerParams
from salt_amd.fpga_export import (channel_thresholds, conv_weight_lines, decay_lines, hex_line,
                                  threshold_lines, write_conv_layer_mem)
from salt_amd.quant.codes import (apply_decay_table_int, build_decay_table_int, iv_from_measurement,
                                  iv_layer, max_weight_code, quantize_to_int,
                                  round_half_away_from_zero, v_th_to_int, waste)
from salt_amd.quant.convert import (LayerQuantSpec, build_quantized_params, iv_per_channel,
                                    weight_codes)
from salt_amd.quant.ptq import (fake_quantize_tensor, percentile_abs_threshold,
                                quantization_error, quantize_params)

# --------------------------------------------------------------------- codes


def test_quantize_to_int_codes_and_fake_quantize_agree():
    x = np.random.default_rng(2).uniform(-5.0, 5.0, 200).astype(np.float32)
    x_hat, scale_a = fake_quantize_tensor(x, bits=8)
    q, scale_b = quantize_to_int(x, bits=8)
    assert q.dtype == np.int32 and int(np.abs(q).max()) == max_weight_code(8)
    assert float(scale_a) == float(scale_b) == np.float32(np.abs(x).max()) / np.float32(127)
    assert np.allclose(q * scale_b, x_hat, atol=1e-5)
    # the largest magnitude maps to the largest code; codes are the nearest levels
    assert np.all(np.abs(x / scale_b - q) <= 0.5 + 1e-4)


def test_quantize_to_int_axis_threshold_and_zero_channels():
    x = np.array([[0.0, 0.0], [1.0, -3.0]], np.float32)
    q, scale = quantize_to_int(x, bits=3, axis=0)           # max code 3
    assert scale.shape == (2, 1) and scale[0, 0] == np.float32(1 / 3)  # all-zero row -> threshold 1
    assert q.tolist() == [[0, 0], [1, -3]]
    q, _ = quantize_to_int(np.array([2.0, -9.0], np.float32), bits=4, threshold=1.0)
    assert q.tolist() == [7, -7]                            # clipped at +-threshold
    with pytest.raises(ValueError):
        quantize_to_int(x, bits=1)


def test_max_weight_code():
    assert max_weight_code(8) == 127 and max_weight_code(4) == 7


def test_apply_decay_table_int_three_regimes():
    """test_quant_codes.py:84-93: table(f_a=4, tau=4), dt [0, 1, 2, 3, 60]."""
    table = build_decay_table_int(4, 4.0)
    a, ident = apply_decay_table_int(np.array([0.0, 1.0, 2.0, 3.0, 60.0]), table)
    assert ident.tolist() == [True, False, False, False, False]
    assert a[1:].tolist() == [12, 9, 7, 0]
    with pytest.raises(ValueError, match="整數"):
        apply_decay_table_int(np.array([1.5]), table)
    with pytest.raises(ValueError, match="2\\^31"):
        apply_decay_table_int(np.array([2.0 ** 31]), table)


def test_iv_formulas():
    assert iv_from_measurement(M=2.0, T_c=1.0, b=8) == 9
    i_V = iv_from_measurement(M=4.0, T_c=127.0, b=8)
    assert i_V == 4 and 2 ** (i_V - 1) > 4
    with pytest.raises(ValueError):
        iv_from_measurement(M=0.0, T_c=1.0, b=8)
    assert iv_layer([3, 5, 4]) == 5 and waste(5, [3, 5, 4]) == [2, 0, 1]


def test_round_half_away_from_zero():
    assert round_half_away_from_zero(np.array([0.4, 0.6, -0.4, -0.6, 0.0])).tolist() == \
        [0.0, 1.0, -0.0, -1.0, 0.0]
    assert round_half_away_from_zero(np.array([2.5, -2.5, 0.5, -1.5])).tolist() == [3, -3, 1, -2]


def test_v_th_to_int():
    assert int(v_th_to_int(v_th=1.95, s_c=0.3, f_V=2, i_V=8)) == 26
    assert int(v_th_to_int(v_th=2.5, s_c=1.0, f_V=0, i_V=8)) == 3   # tie away from zero
    with pytest.raises(ValueError):
        v_th_to_int(v_th=1e9, s_c=0.03, f_V=10, i_V=13)
    assert int(v_th_to_int(v_th=7.0, s_c=1.0, f_V=0, i_V=4)) == 7
    with pytest.raises(ValueError):
        v_th_to_int(v_th=8.0, s_c=1.0, f_V=0, i_V=4)


# --------------------------------------------------------------------- ptq


def test_percentile_threshold_and_error_statistics():
    w = np.array([[0.375, 0.125], [-1.0, 0.25]], np.float32)
    assert percentile_abs_threshold(w, 50.0, axis=0).ravel().tolist() == [0.25, 0.625]
    assert float(percentile_abs_threshold(w, 100.0, axis=None)) == 1.0
    e = quantization_error(w, w)
    assert e["mse"] == 0.0 and e["sqnr_db"] == float("inf")
    e = quantization_error(np.array([1.0, -1.0], np.float32), np.array([0.5, -1.0], np.float32))
    assert e["mse"] == 0.125 and e["max_abs_err"] == 0.5
    assert e["sqnr_db"] == pytest.approx(10 * np.log10(8.0))
    (w_hat,) = quantize_params([w], bits=4)
    assert np.allclose(w_hat, [[0.375, 2 * 0.375 / 7], [-1.0, 2 / 7]])


# --------------------------------------------------------------------- convert

CONV = ConvLayer(name="conv", ic=2, h_in=2, w_in=2, oc=2, k=1, s=1, p=0, init_k=5.0,
                 tau=16.0, v_th=1.0, chunk_size=1, max_queue_len=8, max_out_spikes=64)
FC = FCLayer(name="out", n_in=8, n_out=2, init_k=5.0, tau=16.0, v_th=1e9)
CONV_W = np.array([0.375, 0.125, -1.0, 0.25], np.float32).reshape(2, 2, 1, 1)
FC_W = np.linspace(-0.5, 0.3, 16, dtype=np.float32).reshape(2, 8)


def test_weight_codes_hand_computations():
    """test_quant_convert.py:23-46."""
    q, scale = weight_codes(CONV_W, LayerQuantSpec(bits=4, f_a=8, f_V=4))
    assert q.dtype == np.int32 and q.reshape(2, 2).tolist() == [[7, 2], [-7, 2]]
    assert np.allclose(scale, [0.375 / 7, 1 / 7])
    q, scale = weight_codes(CONV_W, LayerQuantSpec(bits=4, f_a=8, f_V=4, per_channel=False))
    assert q.reshape(2, 2).tolist() == [[3, 1], [-7, 2]] and np.allclose(scale, [1 / 7, 1 / 7])
    _, scale = weight_codes(CONV_W, LayerQuantSpec(bits=4, f_a=8, f_V=4, clip_percentile=50.0))
    assert float(scale[1]) == pytest.approx(0.625 / 7)


def test_iv_per_channel():
    assert iv_per_channel(np.array([2.0, 0.5]), np.array([0.375 / 7, 1 / 7]), bits=4) == [7, 3]
    with pytest.raises(ValueError):
        iv_per_channel(np.array([2.0, 0.5, 1.0]), np.array([0.1, 0.2]), bits=4)


def _build(fc_spec):
    specs = [LayerQuantSpec(bits=4, f_a=8, f_V=4), fc_spec]
    return build_quantized_params([CONV, FC], (CONV_W, FC_W), specs,
                                  [np.array([2.0, 0.5]), np.array([3.0, 1.0])])


def test_build_quantized_params():
    """test_quant_convert.py:67-93."""
    conv_p, _ = _build(LayerQuantSpec(bits=4, f_a=8, f_V=4, fires=False))
    assert conv_p.i_V == 7
    assert np.allclose(conv_p.scale, [0.375 / 7] * 4 + [1 / 7] * 4)
    assert conv_p.v_th_int.tolist() == [299] * 4 + [112] * 4
    assert np.array_equal(conv_p.decay_table_int, build_decay_table_int(8, 16.0))
    assert (conv_p.f_a, conv_p.f_V) == (8, 4)
    _, fc_p = _build(LayerQuantSpec(bits=4, f_a=8, f_V=4, per_channel=False, fires=False))
    assert fc_p.v_th_int is None and fc_p.scale.shape == (2,) and fc_p.scale[0] == fc_p.scale[1]
    with pytest.raises(ValueError):
        build_quantized_params([CONV, FC], (CONV_W, FC_W), [LayerQuantSpec(4, 8, 4)],
                               [np.array([2.0, 0.5]), np.array([3.0, 1.0])])


# --------------------------------------------------------------------- FPGA export


def test_hex_lines():
    assert hex_line(5, 7) == "05" and hex_line(0x1fd, 9) == "1fd" and hex_line(0, 1) == "0"
    for value, width in [(128, 7), (-1, 7), (0, 0)]:
        with pytest.raises(ValueError):
            hex_line(value, width)


def test_weight_words():
    """test_fpga_export.py:24-62."""
    assert conv_weight_lines(np.array([3, -1, 0, -7]).reshape(1, 1, 2, 2), 4) == ["90f3"]
    q = (10 * np.arange(2)[:, None] + np.arange(3)[None, :]).reshape(2, 3, 1, 1)
    assert conv_weight_lines(q, 7) == ["00", "01", "02", "0a", "0b", "0c"]
    assert conv_weight_lines(np.full((1, 1, 3, 3), -1), 7) == ["7fffffffffffffff"]
    q = np.zeros((1, 1, 3, 3), np.int32)
    q[0, 0, 2, 2] = -63
    assert conv_weight_lines(q, 7) == ["4100000000000000"]
    assert conv_weight_lines(np.full((1, 1, 1, 1), -64), 7) == ["40"]
    for code in (64, -65):
        with pytest.raises(ValueError):
            conv_weight_lines(np.full((1, 1, 1, 1), code), 7)
    for shape in [(1, 1, 3), (1, 1, 3, 2)]:
        with pytest.raises(ValueError):
            conv_weight_lines(np.zeros(shape, np.int32), 7)


def test_thresholds_and_decay_lines():
    assert channel_thresholds(np.array([5, 5, 5, -3, -3, -3]), 2).tolist() == [5, -3]
    assert channel_thresholds(np.array(7), 3).tolist() == [7, 7, 7]
    with pytest.raises(ValueError, match=r"\[1\]"):
        channel_thresholds(np.array([5, 5, 5, -3, -2, -3]), 2)
    with pytest.raises(ValueError):
        channel_thresholds(np.array([5, 5, 5]), 2)
    assert threshold_lines([5, -3], 9) == ["005", "1fd"]
    for v in (256, -257):
        with pytest.raises(ValueError):
            threshold_lines([v], 9)
    assert decay_lines([60, 56, 1], 6) == ["3c", "38", "01"]
    for v in (64, -1):
        with pytest.raises(ValueError):
            decay_lines([v], 6)


LAYER = ConvLayer(name="conv1", ic=2, h_in=5, w_in=5, oc=3, k=3, s=2, p=1, init_k=5.0)


def _layer_params(**changes):
    p = QuantizedLayerParams(q=np.random.default_rng(0).integers(-63, 64, size=(3, 2, 3, 3)),
                             decay_table_int=np.array([60, 56, 53]),
                             v_th_int=np.repeat(np.array([24, 35, 63]), 9),
                             scale=np.ones(27, np.float32), f_a=6, f_V=0, i_V=9)
    return p._replace(**changes)


def test_write_conv_layer_mem(tmp_path):
    params = _layer_params()
    paths = write_conv_layer_mem(tmp_path, LAYER, params, 7)
    assert paths == {k: tmp_path / f"conv1_{k}.mem" for k in ("weight", "threshold", "decay")}
    assert paths["weight"].read_text().splitlines() == conv_weight_lines(params.q, 7)
    assert paths["threshold"].read_text() == "018\n023\n03f\n"
    assert paths["decay"].read_text() == "3c\n38\n35\n"


@pytest.mark.parametrize("changes", [{"q": np.zeros((3, 2, 2, 2), np.int32)}, {"v_th_int": None},
                                     {"v_th_int": np.full(12, 24)}])
def test_write_conv_layer_mem_rejects_before_writing(tmp_path, changes):
    with pytest.raises(ValueError):
        write_conv_layer_mem(tmp_path, LAYER, _layer_params(**changes), 7)
    assert list(tmp_path.iterdir()) == []
