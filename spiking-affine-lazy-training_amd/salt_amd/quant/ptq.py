"""Post-training weight quantisation helpers (salt_core/quant/ptq.py): symmetric,
zero-point-free linear quantisation, fake-quantised weights and error statistics.
float32 numpy."""
from __future__ import annotations

from collections.abc import Sequence
from typing import TypedDict

import numpy as np

from salt_amd.quant.codes import _f32, quantize_to_int


def fake_quantize_tensor(x, bits: int, *, axis: int | None = None, threshold=None
                         ) -> tuple[np.ndarray, np.ndarray]:
    """(q * scale, scale) of quantize_to_int: the weights as the integer model sees them,
    back on the float scale (ptq.py:13-22)."""
    q, scale = quantize_to_int(x, bits, axis=axis, threshold=threshold)
    return (q.astype(np.float32) * scale).astype(np.float32), scale


class QuantizationError(TypedDict):
    mse: float
    max_abs_err: float
    sqnr_db: float


def quantization_error(x, x_hat) -> QuantizationError:
    """MSE, max |error| and signal-to-quantisation-noise ratio in dB (ptq.py:32-45)."""
    x, x_hat = _f32(x), _f32(x_hat)
    err = x - x_hat
    mse = float(np.mean(err ** 2))
    signal = float(np.mean(x ** 2))
    return {"mse": mse, "max_abs_err": float(np.max(np.abs(err))),
            "sqnr_db": float("inf") if mse <= 0.0 else 10.0 * float(np.log10(signal / mse))}


def percentile_abs_threshold(x, percentile: float, axis: int | None) -> np.ndarray:
    """The percentile of |x| (linear interpolation) as a clip level, one per position of
    `axis` with the other axes kept as 1 (ptq.py:48-62); 100 = max |x|."""
    abs_x = np.abs(_f32(x))
    if axis is None:
        return np.asarray(np.percentile(abs_x, percentile), dtype=np.float32)
    moved = np.moveaxis(abs_x, axis, 0)
    thresh = np.percentile(moved.reshape(moved.shape[0], -1), percentile, axis=1)
    shape = [1] * abs_x.ndim
    shape[axis] = -1
    return np.asarray(thresh, dtype=np.float32).reshape(shape)


def quantize_params(params: Sequence, *, bits: int, per_channel: bool = True,
                    clip_percentile: float = 100.0) -> tuple[np.ndarray, ...]:
    """Every layer's weights fake-quantised (ptq.py:65-80)."""
    out = []
    for w in params:
        axis = 0 if per_channel else None
        threshold = percentile_abs_threshold(w, clip_percentile, axis=axis)
        out.append(fake_quantize_tensor(w, bits, axis=axis, threshold=threshold)[0])
    return tuple(out)
