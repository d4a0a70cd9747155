"""Literal NumPy restatement of salt_core/quant's queue formulation (test infrastructure
only; small inputs only).

Where salt_oracle.c restates the path event by event, this module follows the
reference's own mechanism step for step: build the per-neuron queue structure
(salt_core/connectivity/{fc,conv}.py), look up decay codes
(salt_core/quant/codes.py:87-105), gather weight codes, scan every queue column for
every neuron (salt_core/quant/scan.py:97-132, with the reference's hi/lo split
multiply in int32), and extract the spike stream with nonzero + stable sort
(salt_core/stream.py:24-100).  The two restatements share no code; tests run both on
the same inputs.

JAX index semantics are reproduced where the reference relies on them: negative
dynamic indices wrap once, out-of-range gathers clamp (_jax_take).
"""
from __future__ import annotations

import numpy as np

PAD_TIME = np.float32(1e12)  # salt_core/stream.py:13
MAX_SHIFT_BITS = 15          # salt_core/quant/fixed_point.py:15
MAX_REGISTER_BITS = 30       # salt_core/quant/fixed_point.py:17


def _jax_take(arr: np.ndarray, idx, axis: int = 0) -> np.ndarray:
    """Gather with JAX's rules for dynamic indices: one wrap of negatives, then clamp."""
    idx = np.asarray(idx)
    n = arr.shape[axis]
    idx = np.where(idx < 0, idx + n, idx)
    idx = np.clip(idx, 0, n - 1)
    return np.take(arr, idx, axis=axis)


# ---------------------------------------------------------------- fixed point

def round_shift(x: np.ndarray, shift_bits: int, round_mode: str) -> np.ndarray:
    """salt_core/quant/fixed_point.py:32-44 (int32 arithmetic)."""
    if round_mode not in ("round", "truncate"):
        raise ValueError(round_mode)
    x = np.asarray(x, dtype=np.int32)
    if shift_bits == 0:
        return x
    if round_mode == "round":
        x = (x + np.int32(1 << (shift_bits - 1))).astype(np.int32)
    return (x >> shift_bits).astype(np.int32)


def wide_mul_shift(a: np.ndarray, v: np.ndarray, shift_bits: int, round_mode: str) -> np.ndarray:
    """salt_core/quant/fixed_point.py:47-65: the hi/lo split, every product in int32."""
    if shift_bits > MAX_SHIFT_BITS:
        raise ValueError("shift_bits above MAX_SHIFT_BITS")
    a = np.asarray(a, dtype=np.int32)
    v = np.asarray(v, dtype=np.int32)
    hi = v >> shift_bits
    lo = v & np.int32((1 << shift_bits) - 1)
    with np.errstate(over="ignore"):
        return (a * hi + round_shift(a * lo, shift_bits, round_mode)).astype(np.int32)


def fit_to_bits(x: np.ndarray, total_bits: int, overflow_mode: str) -> tuple[np.ndarray, np.ndarray]:
    """salt_core/quant/fixed_point.py:68-90."""
    if overflow_mode not in ("wrap", "saturate"):
        raise ValueError(overflow_mode)
    if total_bits > MAX_REGISTER_BITS:
        raise ValueError("total_bits above MAX_REGISTER_BITS")
    x = np.asarray(x, dtype=np.int64)
    half = 1 << (total_bits - 1)
    overflowed = (x < -half) | (x >= half)
    if overflow_mode == "saturate":
        return np.clip(x, -half, half - 1).astype(np.int32), overflowed
    masked = x & ((1 << total_bits) - 1)
    return np.where(masked >= half, masked - (1 << total_bits), masked).astype(np.int32), overflowed


def apply_decay_table_int(delta_t: np.ndarray, table_int: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """salt_core/quant/codes.py:87-105 (float32 dt -> saturating int32 -> clipped gather)."""
    dt = np.asarray(delta_t, dtype=np.float32).astype(np.float64)
    dt = np.clip(dt, -2.0 ** 31, 2.0 ** 31 - 1).astype(np.int64)
    table_int = np.asarray(table_int, dtype=np.int32)
    n = table_int.shape[0]
    idx = np.clip(dt - 1, 0, n - 1)
    gathered = table_int[idx]
    a_int = np.where(dt > n, 0, gathered).astype(np.int32)
    return a_int, dt == 0


def run_layer(a_int, is_identity, q_int, v_th_int, *, f_a, f_V, i_V,
              round_mode="round", overflow_mode="wrap") -> dict:
    """salt_core/quant/scan.py:65-80, 97-132: one scan step per queue column, all
    neurons at once; process_event (scan.py:22-52) inlined."""
    n, steps = a_int.shape
    vth = None if v_th_int is None else np.broadcast_to(
        np.asarray(v_th_int).astype(np.int64).astype(np.int32), (n,))
    v = np.zeros(n, np.int32)
    vmin = np.zeros(n, np.int32)
    vmax = np.zeros(n, np.int32)
    spike_mask = np.zeros((n, steps), bool)
    overflowed = np.zeros((n, steps), bool)
    v_steps = np.zeros((n, steps), np.int32)
    for t in range(steps):
        decayed_active = wide_mul_shift(a_int[:, t], v, f_a, round_mode)
        decayed = np.where(is_identity[:, t], v, decayed_active).astype(np.int32)
        with np.errstate(over="ignore"):
            unfitted = (decayed + q_int[:, t].astype(np.int32) * np.int32(1 << f_V)).astype(np.int32)
        fitted, ovf = fit_to_bits(unfitted, i_V + f_V, overflow_mode)
        if vth is None:
            spiked = np.zeros(n, bool)
            v = fitted
        else:
            spiked = fitted >= vth
            v = np.where(spiked, 0, fitted).astype(np.int32)
        spike_mask[:, t] = spiked
        overflowed[:, t] = ovf
        v_steps[:, t] = v
        vmin = np.minimum(vmin, unfitted)
        vmax = np.maximum(vmax, unfitted)
    return {"spike_mask": spike_mask,
            "spike_event_idx": np.broadcast_to(np.arange(steps), (n, steps)),
            "v_final": v, "overflowed": overflowed, "v_unfitted_min": vmin,
            "v_unfitted_max": vmax, "v_steps": v_steps}


# ---------------------------------------------------------------- FC queue

def build_fc_structure(event_times, event_source_idx, n_real_events) -> dict:
    """salt_core/connectivity/fc.py:20-33."""
    t = np.asarray(event_times, dtype=np.float32)
    gap = np.diff(t, prepend=np.zeros(1, np.float32)).astype(np.float32)
    is_real = np.arange(t.shape[0]) < int(n_real_events)
    return {"delta_t": np.where(is_real, gap, np.float32(0.0)).astype(np.float32),
            "source_idx": np.asarray(event_source_idx), "n_real_events": int(n_real_events)}


def fc_weight_codes(structure: dict, q: np.ndarray) -> np.ndarray:
    """salt_core/connectivity/fc.py:54-61."""
    is_real = np.arange(structure["delta_t"].shape[0]) < structure["n_real_events"]
    gathered = _jax_take(np.asarray(q).astype(np.int64).astype(np.int32),
                         structure["source_idx"], axis=1)
    return np.where(is_real[None, :], gathered, 0).astype(np.int32)


# ---------------------------------------------------------------- conv queue

def _axis_candidates(i, K, S, P, N, O_max):
    """salt_core/connectivity/conv.py:15-29."""
    o_min = (i + P - K + 1 + S - 1) // S
    upper = (i + P) // S
    r = np.arange(N)
    o = o_min[:, None] + r[None, :]
    valid = (o <= upper[:, None]) & (o >= 0) & (o < O_max)
    k = i[:, None] - o * S + P
    return o, valid, k


def unravel_conv_source(src, H_in, W_in):
    """salt_core/connectivity/conv.py:32-43."""
    src = np.asarray(src, dtype=np.int64)
    hw = H_in * W_in
    return src % hw % W_in, src % hw // W_in, src // hw


def _compress_candidates(n_flat, j_flat, n_out_spatial, max_queue_len, n_events):
    """salt_core/connectivity/conv.py:57-99 (stable lexsort, segmented rank, trash row)."""
    order = np.lexsort((j_flat, n_flat))
    sorted_n, sorted_j = n_flat[order], j_flat[order]
    C = n_flat.shape[0]
    idx = np.arange(C)
    is_start = np.concatenate([[True], sorted_n[1:] != sorted_n[:-1]]) if C else np.zeros(0, bool)
    last_start = np.maximum.accumulate(np.where(is_start, idx, -1)) if C else idx
    local_rank = idx - last_start
    invalid = sorted_n >= n_out_spatial
    safe_n = np.where(invalid, n_out_spatial, sorted_n)
    safe_rank = np.where((local_rank >= max_queue_len) | invalid, max_queue_len, local_rank)
    l2g = np.full((n_out_spatial + 1, max_queue_len + 1), n_events, np.int64)
    l2g[safe_n, safe_rank] = sorted_j
    n_real = np.zeros(n_out_spatial + 1, np.int64)
    np.maximum.at(n_real, safe_n, np.where(invalid, 0, local_rank + 1))
    return l2g[:n_out_spatial, :max_queue_len], n_real[:n_out_spatial]


def _delta_t_three_regimes(t_gathered, n_real, global_last_time):
    """salt_core/connectivity/conv.py:102-125 (float32)."""
    n_out, mql = t_gathered.shape
    col = np.arange(mql)[None, :]
    nr = n_real[:, None]
    dt_real = np.diff(t_gathered, axis=1, prepend=np.zeros((n_out, 1), np.float32)).astype(np.float32)
    last_col = np.clip(n_real - 1, 0, mql - 1)
    t_last_real = np.take_along_axis(t_gathered, last_col[:, None], axis=1)[:, 0]
    dt_catch = (np.float32(global_last_time) - t_last_real).astype(np.float32)
    return np.where(col < nr, dt_real, np.where(col == nr, dt_catch[:, None], np.float32(0.0))).astype(np.float32)


def build_conv_structure(event_times, x, y, c, k, s, p, h_out, w_out, max_queue_len, n_real_events):
    """salt_core/connectivity/conv.py:128-172."""
    t = np.asarray(event_times, dtype=np.float32)
    x, y, c = (np.asarray(a, dtype=np.int64) for a in (x, y, c))
    n_events = t.shape[0]
    n_input = int(n_real_events)
    N = (k - 1) // s + 1
    n_spatial = h_out * w_out
    o_y, valid_y, _ = _axis_candidates(y, k, s, p, N, h_out)
    o_x, valid_x, _ = _axis_candidates(x, k, s, p, N, w_out)
    is_real = np.arange(n_events) < n_input
    valid = valid_y[:, :, None] & valid_x[:, None, :] & is_real[:, None, None]
    n2d = o_y[:, :, None] * w_out + o_x[:, None, :]
    j2d = np.broadcast_to(np.arange(n_events)[:, None, None], (n_events, N, N))
    n_flat = np.where(valid, n2d, n_spatial).reshape(-1)
    l2g, n_real_pos = _compress_candidates(n_flat, j2d.reshape(-1), n_spatial, max_queue_len, n_events)
    event_j = np.minimum(l2g, n_input - 1)
    delta_t = _delta_t_three_regimes(_jax_take(t, event_j), n_real_pos, _jax_take(t, n_input - 1))
    oy_grid = (np.arange(n_spatial) // w_out)[:, None]
    ox_grid = (np.arange(n_spatial) % w_out)[:, None]
    tap_ky = np.clip(_jax_take(y, event_j) - oy_grid * s + p, 0, k - 1)
    tap_kx = np.clip(_jax_take(x, event_j) - ox_grid * s + p, 0, k - 1)
    return {"local_to_global_j": l2g, "n_real_events": n_real_pos, "delta_t": delta_t,
            "tap_c": _jax_take(c, event_j), "tap_ky": tap_ky, "tap_kx": tap_kx,
            "n_input_events": n_input}


def tile_channels(values: np.ndarray, oc: int) -> np.ndarray:
    """salt_core/connectivity/conv.py:221-225."""
    return np.broadcast_to(values[None], (oc, *values.shape)).reshape(oc * values.shape[0], *values.shape[1:])


def conv_weight_codes(structure: dict, q: np.ndarray) -> np.ndarray:
    """salt_core/connectivity/conv.py:175-184, 209-218."""
    q = np.asarray(q).astype(np.int64).astype(np.int32)
    oc, ic = q.shape[0], q.shape[1]
    n_spatial, mql = structure["delta_t"].shape
    tap_c = np.clip(structure["tap_c"], 0, ic - 1)
    taps = q[:, tap_c, structure["tap_ky"], structure["tap_kx"]]  # (oc, n_spatial, mql)
    real = np.arange(mql)[None, :] < structure["n_real_events"][:, None]
    return np.where(real[None], taps, 0).astype(np.int32).reshape(oc * n_spatial, mql)


# ---------------------------------------------------------------- stream extraction

def _select_spikes(spike_mask, spike_event_idx, max_total_spikes):
    """salt_core/stream.py:49-64."""
    n, steps = spike_mask.shape
    if max_total_spikes is None:
        max_total_spikes = n * steps
    nz_n, nz_t = np.nonzero(spike_mask)
    neuron_idx = np.zeros(max_total_spikes, np.int64)
    step_idx = np.zeros(max_total_spikes, np.int64)
    m = min(max_total_spikes, nz_n.shape[0])
    neuron_idx[:m], step_idx[:m] = nz_n[:m], nz_t[:m]
    n_real = int(spike_mask.sum())
    return neuron_idx, spike_event_idx[neuron_idx, step_idx], n_real, max_total_spikes


def _pack_stream(neuron_idx, global_event_idx, input_event_times, n_real, max_total):
    """salt_core/stream.py:24-46."""
    t = np.asarray(input_event_times, dtype=np.float32)
    n_events = t.shape[0]
    real = np.arange(max_total) < n_real
    raw_times = _jax_take(t, np.minimum(global_event_idx, n_events - 1))
    order = np.argsort(np.where(real, global_event_idx, n_events), kind="stable")
    out_times = np.where(real, raw_times, PAD_TIME).astype(np.float32)[order]
    return out_times, neuron_idx[order].astype(np.int32), n_real


# ---------------------------------------------------------------- layers

def fc_forward(q, table, v_th, f_a, f_V, i_V, times, src, n_real, max_out_spikes,
               round_mode="round", overflow_mode="wrap") -> dict:
    """salt_core/layers/fc.py:84-124 under QuantBackend (quant/backend.py:31-53)."""
    st = build_fc_structure(times, src, n_real)
    q_int = fc_weight_codes(st, q)
    a_int, ident = apply_decay_table_int(np.broadcast_to(st["delta_t"], q_int.shape), table)
    r = run_layer(a_int, ident, q_int, v_th, f_a=f_a, f_V=f_V, i_V=i_V,
                  round_mode=round_mode, overflow_mode=overflow_mode)
    nid, gj, nr, mo = _select_spikes(r["spike_mask"], r["spike_event_idx"], max_out_spikes)
    ot, os_, n = _pack_stream(nid, gj, times, nr, mo)
    r.update(out_times=ot, out_src=os_, out_n=n, needed_queue=0)
    return r


def conv_forward(q, table, v_th, f_a, f_V, i_V, times, src, n_real, max_out_spikes, *,
                 ic, h_in, w_in, k, s, p, max_queue_len, round_mode="round",
                 overflow_mode="wrap") -> dict:
    """salt_core/layers/conv.py:124-175 under QuantBackend."""
    q = np.asarray(q)
    oc = q.shape[0]
    h_out = (h_in + 2 * p - k) // s + 1
    w_out = (w_in + 2 * p - k) // s + 1
    x, y, c = unravel_conv_source(src, h_in, w_in)
    st = build_conv_structure(times, x, y, c, k, s, p, h_out, w_out, max_queue_len, n_real)
    q_int = conv_weight_codes(st, q)
    a_int, ident = apply_decay_table_int(tile_channels(st["delta_t"], oc), table)
    r = run_layer(a_int, ident, q_int, v_th, f_a=f_a, f_V=f_V, i_V=i_V,
                  round_mode=round_mode, overflow_mode=overflow_mode)
    l2g = tile_channels(st["local_to_global_j"], oc)
    nid, col, nr, mo = _select_spikes(r["spike_mask"], r["spike_event_idx"], max_out_spikes)
    gj = l2g[nid, np.minimum(col, max_queue_len - 1)]
    ot, os_, n = _pack_stream(nid, gj, times, nr, mo)
    r.update(out_times=ot, out_src=os_, out_n=n,
             needed_queue=int(st["n_real_events"].max()) + 1 if st["n_real_events"].size else 1)
    return r
