"""Float weights + a quantisation spec -> QuantizedLayerParams per layer
(salt_core/quant/convert.py): weight codes and per-channel steps s_c, the register's
integer bits from measured membrane magnitudes, integer thresholds and decay tables."""
from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import numpy as np

from salt_amd.quant.codes import (build_decay_table_int, iv_from_measurement, iv_layer,
                                  max_weight_code, quantize_to_int, v_th_to_int)
from salt_amd.quant.fixed_point import OverflowMode
from salt_amd.quant.params import QuantizedLayerParams
from salt_amd.quant.ptq import percentile_abs_threshold


class LayerQuantSpec(NamedTuple):
    """One layer's quantisation spec (convert.py:21-29)."""
    bits: int                        # weight code width b
    f_a: int                         # fraction bits of the decay code
    f_V: int                         # fraction bits of the register
    per_channel: bool = True         # False: one s_c for the whole layer
    fires: bool = True               # False: no threshold (membrane-regression output layer)
    clip_percentile: float = 100.0   # clip level = this percentile of |w| (100 = max)
    overflow_mode: OverflowMode | str = OverflowMode.WRAP


def weight_codes(w, spec: LayerQuantSpec) -> tuple[np.ndarray, np.ndarray]:
    """(q int32 shaped like w, s_c per output channel (axis 0)) (convert.py:32-42)."""
    w = np.asarray(w)
    axis = 0 if spec.per_channel else None
    threshold = percentile_abs_threshold(w, spec.clip_percentile, axis=axis)
    q, scale = quantize_to_int(w, bits=spec.bits, axis=axis, threshold=threshold)
    return q, np.broadcast_to(np.asarray(scale).reshape(-1), (w.shape[0],)).copy()


def iv_per_channel(v_abs_max, scale, bits: int) -> list[int]:
    """Per-channel i_V from the measured magnitudes M and steps s_c (convert.py:45-58)."""
    v_abs_max = np.asarray(v_abs_max)
    clip_threshold = np.asarray(scale) * max_weight_code(bits)
    if v_abs_max.shape != clip_threshold.shape:
        raise ValueError(f"v_abs_max 形狀 {v_abs_max.shape} 跟 scale 形狀 "
                         f"{clip_threshold.shape} 不一樣")
    return [iv_from_measurement(float(m), float(t), bits)
            for m, t in zip(v_abs_max, clip_threshold)]


def build_quantized_params(layers: Sequence, float_params: Sequence, specs: Sequence[LayerQuantSpec],
                           v_abs_max: Sequence) -> list[QuantizedLayerParams]:
    """Each layer's QuantizedLayerParams, ready for QuantBackend (convert.py:61-87).
    i_V is the tightest channel's; v_abs_max per layer holds the measured per-channel
    membrane magnitudes M.  Lengths that differ raise ValueError."""
    lengths = {len(layers), len(float_params), len(specs), len(v_abs_max)}
    if len(lengths) != 1:
        raise ValueError(f"layers、float_params、specs、v_abs_max 長度要一樣,拿到 "
                         f"{len(layers)}、{len(float_params)}、{len(specs)}、{len(v_abs_max)}")
    out = []
    for layer, w, spec, m in zip(layers, float_params, specs, v_abs_max):
        q, scale_per_channel = weight_codes(w, spec)
        i_V = iv_layer(iv_per_channel(m, scale_per_channel, spec.bits))
        scale_per_neuron = layer.broadcast_channels(scale_per_channel)
        v_th_int = v_th_to_int(layer.v_th, scale_per_neuron, spec.f_V, i_V) if spec.fires else None
        out.append(QuantizedLayerParams(
            q=q, decay_table_int=build_decay_table_int(spec.f_a, layer.tau), v_th_int=v_th_int,
            scale=scale_per_neuron, f_a=spec.f_a, f_V=spec.f_V, i_V=i_V,
            overflow_mode=spec.overflow_mode))
    return out
