"""Post-training quantisation of float weights (the operations of salt_core/quant/ptq.py):
symmetric, zero-point-free linear codes (codes.quantize_to_int), the weights as the integer
model sees them back on the float scale, clip levels from a percentile of |w|, and the
error statistics of a quantisation.  float32 numpy throughout.
"""
from __future__ import annotations

from collections.abc import Sequence
from typing import TypedDict

import numpy as np

from salt_amd.quant.codes import _f32, quantize_to_int


def percentile_abs_threshold(x, percentile: float, axis: int | None) -> np.ndarray:
    """A clip level: the given percentile of |x| (linear interpolation; 100 = max |x|),
    over the whole tensor (axis None, a scalar) or per position of `axis`, shaped with
    every other axis kept as 1 so that it broadcasts against x."""
    magnitude = np.abs(_f32(x))
    if axis is None:
        return np.asarray(np.percentile(magnitude, percentile), dtype=np.float32)
    others = tuple(a for a in range(magnitude.ndim) if a != axis % magnitude.ndim)
    level = np.percentile(magnitude, percentile, axis=others, keepdims=True)
    return np.asarray(level, dtype=np.float32)


def fake_quantize_tensor(x, bits: int, *, axis: int | None = None, threshold=None
                         ) -> tuple[np.ndarray, np.ndarray]:
    """(x_hat, scale) with x_hat = q * scale for the codes q of quantize_to_int (same
    arguments): the float weights a layer computes with after quantisation."""
    codes, scale = quantize_to_int(x, bits, axis=axis, threshold=threshold)
    return np.multiply(codes, scale, dtype=np.float32), scale


class QuantizationError(TypedDict):
    mse: float
    max_abs_err: float
    sqnr_db: float


def quantization_error(x, x_hat) -> QuantizationError:
    """Mean squared error, largest |error| and signal-to-quantisation-noise ratio (dB;
    inf when x_hat equals x)."""
    ref, approx = _f32(x), _f32(x_hat)
    diff = ref - approx
    noise = float(np.mean(np.square(diff)))
    power = float(np.mean(np.square(ref)))
    return {"mse": noise, "max_abs_err": float(np.abs(diff).max()),
            "sqnr_db": float("inf") if noise <= 0.0 else 10.0 * float(np.log10(power / noise))}


def quantize_params(params: Sequence, *, bits: int, per_channel: bool = True,
                    clip_percentile: float = 100.0) -> tuple[np.ndarray, ...]:
    """Every layer's weights (one array each) fake-quantised: per output channel (axis 0)
    or per tensor, clipped at the clip_percentile of |w|."""
    axis = 0 if per_channel else None

    def one(w):
        level = percentile_abs_threshold(w, clip_percentile, axis=axis)
        return fake_quantize_tensor(w, bits, axis=axis, threshold=level)[0]

    return tuple(one(w) for w in params)
