"""Offline integer constants needed to build parameters: the decay table and its depth
(salt_core/quant/codes.py:63-84).

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


def _round_half_away_from_zero(x: np.ndarray) -> np.ndarray:
    """codes.py:17-23, in the dtype of x."""
    return np.sign(x) * np.floor(np.abs(x) + x.dtype.type(0.5))


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
