"""Offline integer constants (salt_core/quant/codes.py): weight codes, the decay table
and its depth, integer thresholds and the register-width formulas.  float32 arithmetic,
as the reference's (JAX float32) is; floats become codes by rounding half away from zero.

build_decay_table_int follows the reference's float32 arithmetic
((1 - 1/tau) ** dt in float32, round half away from zero, clamp to 2^f_a - 1).  The
reference evaluates the power with XLA's float32 pow, which is not available here, so a
code that lands within one float32 ulp of a .5 tie may differ; decay_table_ties() lists
such entries.  The table is data: a loaded model carries its own (model.npz), and the
kernels use whatever table they are given."""
import math

import numpy as np


def max_weight_code(bits: int) -> int:
    """Largest symmetric code 2^(bits-1) - 1 (codes.py:12-14)."""
    return 2 ** (bits - 1) - 1


def delta_t_max(f_a: int, tau: float) -> int:
    """Largest dt whose decay code is non-zero (codes.py:63-71)."""
    eps = 2.0 ** -(f_a + 1)
    log_base = math.log(1.0 - 1.0 / tau)
    return max(int(math.floor(math.log(eps) / log_base)), 0)


def round_half_away_from_zero(x) -> np.ndarray:
    """sign(x) * floor(|x| + 0.5) in the dtype of x (float32 for Python scalars): 2.5 -> 3,
    -2.5 -> -3 (codes.py:17-23)."""
    x = np.asarray(x)
    if not np.issubdtype(x.dtype, np.floating):
        x = x.astype(np.float32)
    return np.sign(x) * np.floor(np.abs(x) + x.dtype.type(0.5))


_round_half_away_from_zero = round_half_away_from_zero


def _f32(x) -> np.ndarray:
    """x as JAX would hold it: float64 input stays float32 (JAX's default width)."""
    x = np.asarray(x)
    return x.astype(np.float32) if x.dtype != np.float32 else x


def quantize_to_int(x, bits: int, *, axis: int | None = None, threshold=None
                    ) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric linear quantisation (codes.py:30-56): (q int32, scale) with
    scale = threshold / max_weight_code(bits) and q = round(clip(x, +-threshold) / scale).
    threshold: clip level, max |x| (per position of `axis`) when None; <= 0 counts as 1.
    bits < 2 raises ValueError."""
    if bits < 2:
        raise ValueError(f"bits 必須 >= 2,給的是 {bits!r}")
    x = _f32(x)
    if threshold is None:
        if axis is None:
            threshold = np.max(np.abs(x))
        else:
            reduce_axes = tuple(i for i in range(x.ndim) if i != axis)
            threshold = np.max(np.abs(x), axis=reduce_axes, keepdims=True)
    threshold = np.asarray(threshold, dtype=x.dtype)
    threshold = np.where(threshold > 0, threshold, np.ones_like(threshold))
    scale = (threshold / x.dtype.type(max_weight_code(bits))).astype(x.dtype)
    clipped = np.clip(x, -threshold, threshold)
    q = round_half_away_from_zero((clipped / scale).astype(x.dtype)).astype(np.int32)
    return q, scale


def build_decay_table_int(f_a: int, tau: float) -> np.ndarray:
    """Decay codes for dt = 1..delta_t_max(f_a, tau), int32 (codes.py:74-84)."""
    n = delta_t_max(f_a, tau)
    dt = np.arange(1, n + 1, dtype=np.float32)
    base = np.float32(1.0 - 1.0 / tau)
    a_exact = np.power(base, dt, dtype=np.float32)
    code = _round_half_away_from_zero((a_exact * np.float32(2 ** f_a)).astype(np.float32))
    return np.minimum(code, np.float32(2 ** f_a - 1)).astype(np.int32)


def decay_table_ties(f_a: int, tau: float, tol: float = 1e-3) -> np.ndarray:
    """Indices whose exact (float64) a * 2^f_a lies within tol of a .5 tie: the entries
    whose code could depend on the float32 pow implementation."""
    n = delta_t_max(f_a, tau)
    x = (1.0 - 1.0 / tau) ** np.arange(1, n + 1, dtype=np.float64) * 2.0 ** f_a
    frac = x - np.floor(x)
    return np.nonzero(np.abs(frac - 0.5) < tol)[0]


def apply_decay_table_int(delta_t, table_int) -> tuple[np.ndarray, np.ndarray]:
    """(a_int, is_identity) for integer-ms dt (codes.py:87-116): dt = 0 is the identity,
    1 <= dt <= n reads table[dt - 1], dt > n gives 0.  Non-integer dt or dt outside
    [0, 2^31) raises ValueError.  (The kernels do this lookup per event; this host form
    serves the queue-formulation tools.)"""
    delta_t = np.asarray(delta_t)
    if not np.all(delta_t == np.floor(delta_t)):
        bad = delta_t[delta_t != np.floor(delta_t)]
        raise ValueError(f"Δt 必須是整數毫秒,有非整數值,例如 {bad[:5].tolist()}")
    out_of_range = (delta_t < 0) | (delta_t >= 2.0 ** 31)
    if np.any(out_of_range):
        raise ValueError(f"Δt 必須在 [0, 2^31) 裡,有超出範圍的值,例如 "
                         f"{delta_t[out_of_range][:5].tolist()}")
    dt = delta_t.astype(np.int64)
    table = np.asarray(table_int).astype(np.int32)
    n = table.shape[0]
    gathered = table[np.clip(dt - 1, 0, n - 1)]
    return np.where(dt > n, 0, gathered).astype(np.int32), dt == 0


def v_th_to_int(v_th, s_c, f_V: int, i_V: int) -> np.ndarray:
    """Integer threshold round(v_th / s_c * 2^f_V) in float32 (codes.py:119-136); a code
    outside the (i_V + f_V)-bit register raises ValueError (a layer that never fires
    takes v_th_int = None instead)."""
    v = (_f32(v_th) / _f32(s_c)).astype(np.float32)
    code = round_half_away_from_zero((v * np.float32(2 ** f_V)).astype(np.float32))
    half = 2 ** (i_V + f_V - 1)
    out_of_range = (code < -half) | (code > half - 1)
    if np.any(out_of_range):
        raise ValueError(
            f"整數門檻超出 i_V={i_V}、f_V={f_V} 暫存器的範圍 [{-half}, {half - 1}],"
            f"例如 {np.atleast_1d(code)[np.atleast_1d(out_of_range)][:5].tolist()}。"
            "這層不 fire 的話用 v_th_int=None。")
    return code.astype(np.int32)


def iv_from_measurement(M: float, T_c: float, b: int) -> int:
    """One channel's integer bits i_V = floor(log2(M * (2^(b-1) - 1) / T_c)) + 2, so that
    2^(i_V - 1) exceeds the measured magnitude (codes.py:142-154).  M <= 0 raises."""
    if M <= 0:
        raise ValueError(f"M 必須 > 0,給的是 {M!r}(死 channel 應該先篩掉,不要呼叫這個函式)")
    x = M * max_weight_code(b) / T_c
    return math.floor(math.log2(x)) + 2


def iv_layer(iv_per_channel: list[int]) -> int:
    """A layer's shared i_V: the largest channel's (codes.py:157-159)."""
    return max(iv_per_channel)


def waste(iv_layer_value: int, iv_per_channel: list[int]) -> list[int]:
    """Bits each channel pays for sharing the layer's i_V (codes.py:162-167)."""
    return [iv_layer_value - v for v in iv_per_channel]
