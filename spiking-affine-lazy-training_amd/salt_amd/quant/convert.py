"""Offline conversion of a float model into the integer path's parameters (the conversion
of salt_core/quant/convert.py): per layer the weight codes q and per-channel steps s_c, the
register's integer bits i_V from measured membrane magnitudes, the integer thresholds and
the decay table, as QuantizedLayerParams.
"""
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
    """How one layer is quantised (field names of salt_core/quant/convert.py:21-29)."""
    bits: int                        # weight code width b
    f_a: int                         # fraction bits of the decay code
    f_V: int                         # fraction bits of the register
    per_channel: bool = True         # False: one step s_c for the whole layer
    fires: bool = True               # False: no threshold (membrane-regression output layer)
    clip_percentile: float = 100.0   # clip level = this percentile of |w| (100: max |w|)
    overflow_mode: OverflowMode | str = OverflowMode.WRAP


def weight_codes(w, spec: LayerQuantSpec) -> tuple[np.ndarray, np.ndarray]:
    """(q, s): int32 codes shaped like w (axis 0 = output channel) and one step per
    output channel (the same step everywhere when the spec is not per channel)."""
    w = np.asarray(w)
    axis = 0 if spec.per_channel else None
    level = percentile_abs_threshold(w, spec.clip_percentile, axis=axis)
    codes, step = quantize_to_int(w, bits=spec.bits, axis=axis, threshold=level)
    per_channel = np.empty(w.shape[0], dtype=np.asarray(step).dtype)
    per_channel[...] = np.asarray(step).reshape(-1)
    return codes, per_channel


def iv_per_channel(v_abs_max, scale, bits: int) -> list[int]:
    """i_V of each channel from its measured membrane magnitude M and step s_c (clip
    level s_c * max_weight_code(bits)); mismatched shapes raise ValueError."""
    measured = np.asarray(v_abs_max)
    clip = np.asarray(scale) * max_weight_code(bits)
    if measured.shape != clip.shape:
        raise ValueError(f"v_abs_max 形狀 {measured.shape} 跟 scale 形狀 {clip.shape} 不一樣")
    return [iv_from_measurement(float(m), float(c), bits) for m, c in zip(measured, clip)]


def _layer_params(layer, w, spec: LayerQuantSpec, v_abs_max) -> QuantizedLayerParams:
    """One layer: i_V is its tightest channel's; steps and thresholds are per neuron."""
    codes, step = weight_codes(w, spec)
    i_V = iv_layer(iv_per_channel(v_abs_max, step, spec.bits))
    step_per_neuron = layer.broadcast_channels(step)
    threshold = v_th_to_int(layer.v_th, step_per_neuron, spec.f_V, i_V) if spec.fires else None
    return QuantizedLayerParams(q=codes, decay_table_int=build_decay_table_int(spec.f_a, layer.tau),
                                v_th_int=threshold, scale=step_per_neuron, f_a=spec.f_a,
                                f_V=spec.f_V, i_V=i_V, overflow_mode=spec.overflow_mode)


def build_quantized_params(layers: Sequence, float_params: Sequence, specs: Sequence[LayerQuantSpec],
                           v_abs_max: Sequence) -> list[QuantizedLayerParams]:
    """Every layer's QuantizedLayerParams (the weights QuantBackend runs): float_params,
    specs and v_abs_max (per layer, the measured per-channel magnitudes M) in layer order;
    sequences of different lengths raise ValueError."""
    if not len(layers) == len(float_params) == len(specs) == len(v_abs_max):
        raise ValueError(f"layers、float_params、specs、v_abs_max 長度要一樣,拿到 "
                         f"{len(layers)}、{len(float_params)}、{len(specs)}、{len(v_abs_max)}")
    return [_layer_params(*args) for args in zip(layers, float_params, specs, v_abs_max)]
