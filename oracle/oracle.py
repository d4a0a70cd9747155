"""Python side of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module.  It wraps liboracle_salt.so (salt_oracle.c, the event-driven restatement of
salt_core/quant) with numpy in/out, and chains layers the way
salt_core/network.py:93-122 (run_network) does.

Geometry and parameters are plain dicts so that the oracle shares no code with the
product package:
    FC:   {"kind": "fc", "n_in": int, "n_out": int}
    conv: {"kind": "conv", "ic", "h_in", "w_in", "oc", "k", "s", "p", "max_queue_len"}
    params: {"q": int array, "table": int array, "v_th": None | int | int array,
             "f_a", "f_V", "i_V", "round_mode": "round"|"truncate",
             "overflow_mode": "wrap"|"saturate"}
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_salt.so")
_lib = None

PAD_TIME = np.float32(1e12)  # salt_core/stream.py:13


class _Geom(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("kind", "n_in", "n_out", "ic", "h_in", "w_in", "oc", "k", "s", "p",
                 "max_queue_len")]


class _QParams(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("table", ctypes.c_void_p), ("n_table", ctypes.c_int32),
                ("v_th", ctypes.c_void_p), ("v_th_kind", ctypes.c_int32),
                ("f_a", ctypes.c_int32), ("f_V", ctypes.c_int32), ("i_V", ctypes.c_int32),
                ("round_mode", ctypes.c_int32), ("overflow_mode", ctypes.c_int32)]


def build() -> str:
    """Compile liboracle_salt.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle_salt.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        i32, f32, p = ctypes.c_int32, ctypes.c_float, ctypes.c_void_p
        _lib.oracle_round_shift.argtypes = [ctypes.c_int64, i32, i32]
        _lib.oracle_round_shift.restype = i32
        _lib.oracle_wide_mul_shift.argtypes = [i32, i32, i32, i32]
        _lib.oracle_wide_mul_shift.restype = i32
        _lib.oracle_fit_to_bits.argtypes = [i32, i32, i32, ctypes.POINTER(i32)]
        _lib.oracle_fit_to_bits.restype = i32
        _lib.oracle_decay_lookup.argtypes = [f32, p, i32, ctypes.POINTER(i32)]
        _lib.oracle_decay_lookup.restype = i32
        _lib.oracle_process_event.argtypes = [i32] * 11 + [ctypes.POINTER(i32)] * 3
        _lib.oracle_process_event.restype = i32
        _lib.oracle_layer_forward.argtypes = [ctypes.POINTER(_Geom), ctypes.POINTER(_QParams),
                                              i32, i32, p, p, p, i32, p, p, p, p, p, p, p, i32]
        _lib.oracle_layer_forward.restype = ctypes.c_int
        _lib.oracle_layer_forward_hashed.argtypes = [ctypes.POINTER(_Geom),
                                                     ctypes.POINTER(_QParams), i32, i32, p, p,
                                                     p, i32, p, p, p, p, p, p, i32]
        _lib.oracle_layer_forward_hashed.restype = ctypes.c_int
        _lib.oracle_stream_hash.argtypes = [p, p, i32, i32]
        _lib.oracle_stream_hash.restype = ctypes.c_uint64
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


_ROUND = {"round": 0, "truncate": 1}
_OVERFLOW = {"wrap": 0, "saturate": 1}


# ---------------------------------------------------------------- primitives

def round_shift(x: int, shift_bits: int, round_mode: str) -> int:
    return lib().oracle_round_shift(int(x), shift_bits, _ROUND[round_mode])


def wide_mul_shift(a: int, v: int, shift_bits: int, round_mode: str) -> int:
    return lib().oracle_wide_mul_shift(int(a), int(v), shift_bits, _ROUND[round_mode])


def fit_to_bits(x: int, total_bits: int, overflow_mode: str) -> tuple[int, bool]:
    ovf = ctypes.c_int32(0)
    v = lib().oracle_fit_to_bits(int(x), total_bits, _OVERFLOW[overflow_mode], ctypes.byref(ovf))
    return v, bool(ovf.value)


def decay_lookup(delta_t: float, table) -> tuple[int, bool]:
    table = np.ascontiguousarray(table, dtype=np.int32)
    ident = ctypes.c_int32(0)
    a = lib().oracle_decay_lookup(float(delta_t), _ptr(table), table.shape[0], ctypes.byref(ident))
    return a, bool(ident.value)


def process_event(v0, a_int, is_identity, q_int, v_th, *, f_a, f_V, i_V,
                  round_mode="round", overflow_mode="wrap") -> dict:
    sp, ovf, u = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    v = lib().oracle_process_event(int(v0), int(a_int), int(bool(is_identity)), int(q_int),
                                   int(v_th is not None), 0 if v_th is None else int(v_th),
                                   f_a, f_V, i_V, _ROUND[round_mode], _OVERFLOW[overflow_mode],
                                   ctypes.byref(sp), ctypes.byref(ovf), ctypes.byref(u))
    return {"v_final": v, "is_spiked": bool(sp.value), "overflowed": bool(ovf.value),
            "v_unfitted": u.value}


def stream_hash(times, src, n: int, cap: int) -> int:
    times = np.ascontiguousarray(times, dtype=np.float32)
    src = np.ascontiguousarray(src, dtype=np.int32)
    return int(lib().oracle_stream_hash(_ptr(times), _ptr(src), int(n), int(cap)))


# ---------------------------------------------------------------- layers

def n_neurons(geom: dict) -> int:
    if geom["kind"] == "fc":
        return geom["n_out"]
    h = (geom["h_in"] + 2 * geom["p"] - geom["k"]) // geom["s"] + 1
    w = (geom["w_in"] + 2 * geom["p"] - geom["k"]) // geom["s"] + 1
    return geom["oc"] * h * w


def layer_forward(geom: dict, params: dict, times, src, n_real, cap: int,
                  nthreads: int = 0, want_stream: bool = True, hashed: bool = False) -> dict:
    """One layer over a batch.  times/src: (B, L); n_real: (B,).  Returns numpy arrays:
    out_times/out_src (B, cap), out_n (B,), v_final/v_min/v_max (B, N), needed_queue (B,).
    hashed: instead of out_times/out_src, out_hash (B,) uint64 -- each stream's
    stream_hash() -- without allocating the (B, cap) output."""
    times = np.ascontiguousarray(times, dtype=np.float32)
    src = np.ascontiguousarray(src, dtype=np.int32)
    n_real = np.ascontiguousarray(n_real, dtype=np.int32).reshape(-1)
    if times.ndim == 1:
        times, src = times[None], src[None]
    B, L = times.shape
    g = _Geom()
    if geom["kind"] == "fc":
        g.kind, g.n_in, g.n_out = 0, geom["n_in"], geom["n_out"]
    else:
        g.kind = 1
        for f in ("ic", "h_in", "w_in", "oc", "k", "s", "p", "max_queue_len"):
            setattr(g, f, int(geom[f]))
    N = n_neurons(geom)
    q = np.ascontiguousarray(np.asarray(params["q"]).astype(np.int64).astype(np.int32))
    table = np.ascontiguousarray(params["table"], dtype=np.int32)
    v_th = params.get("v_th")
    if v_th is None:
        vth_arr, vth_kind = None, 0
    else:
        vth_arr = np.ascontiguousarray(np.asarray(v_th).astype(np.int64).astype(np.int32)).reshape(-1)
        vth_kind = 1 if vth_arr.shape[0] == 1 else 2
        if vth_kind == 2 and vth_arr.shape[0] != N:
            raise ValueError("per-neuron v_th must have one value per neuron")
    qp = _QParams(q=_ptr(q), table=_ptr(table), n_table=table.shape[0], v_th=_ptr(vth_arr),
                  v_th_kind=vth_kind, f_a=params["f_a"], f_V=params["f_V"], i_V=params["i_V"],
                  round_mode=_ROUND[params.get("round_mode", "round")],
                  overflow_mode=_OVERFLOW[params.get("overflow_mode", "wrap")])
    out = {"out_n": np.zeros(B, np.int32), "v_final": np.zeros((B, N), np.int32),
           "v_min": np.zeros((B, N), np.int32), "v_max": np.zeros((B, N), np.int32),
           "needed_queue": np.zeros(B, np.int32)}
    if hashed:
        out["out_hash"] = np.zeros(B, np.uint64)
        rc = lib().oracle_layer_forward_hashed(
            ctypes.byref(g), ctypes.byref(qp), B, L, _ptr(times), _ptr(src), _ptr(n_real), cap,
            _ptr(out["out_n"]), _ptr(out["out_hash"]), _ptr(out["v_final"]), _ptr(out["v_min"]),
            _ptr(out["v_max"]), _ptr(out["needed_queue"]), nthreads)
        if rc != 0:
            raise ValueError("oracle_layer_forward_hashed rejected its arguments")
        return out
    if want_stream:
        out["out_times"] = np.zeros((B, cap), np.float32)
        out["out_src"] = np.zeros((B, cap), np.int32)
    rc = lib().oracle_layer_forward(
        ctypes.byref(g), ctypes.byref(qp), B, L, _ptr(times), _ptr(src), _ptr(n_real), cap,
        _ptr(out.get("out_times")), _ptr(out.get("out_src")), _ptr(out["out_n"]),
        _ptr(out["v_final"]), _ptr(out["v_min"]), _ptr(out["v_max"]), _ptr(out["needed_queue"]),
        nthreads)
    if rc != 0:
        raise ValueError("oracle_layer_forward rejected its arguments")
    return out


def network_forward(layers: list[tuple[dict, dict, int]], times, src, n_real,
                    nthreads: int = 0) -> list[dict]:
    """Chain layers as salt_core/network.py:93-122: each layer's output stream
    (length cap, n_real = total spikes) is the next layer's input.
    layers: [(geom, params, cap)]."""
    results = []
    t, s, n = times, src, n_real
    for geom, params, cap in layers:
        r = layer_forward(geom, params, t, s, n, cap, nthreads=nthreads)
        results.append(r)
        t, s, n = r["out_times"], r["out_src"], r["out_n"]
    return results
