"""ctypes binding of libsalt_hip.so (declarations in include/salt_hip.h).

torch is imported before the library is loaded so that the library binds to the HIP
runtime torch already loaded (same soname): one runtime per process, which is what makes
torch's device pointers and stream handles valid in the library's calls.

There is no fallback: if the library is missing or a call fails, this module raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- must be loaded before libsalt_hip.so, see module docstring

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsalt_hip.so")

SALT_LAYER_FC, SALT_LAYER_CONV = 0, 1
SALT_VTH_NONE, SALT_VTH_SCALAR, SALT_VTH_PER_CHANNEL, SALT_VTH_PER_NEURON = 0, 1, 2, 3
SALT_ROUND, SALT_TRUNCATE = 0, 1
SALT_WRAP, SALT_SATURATE = 0, 1
SALT_STATIC_SCRATCH_BYTES = 64 << 20  # salt_layer_forward_static's per-device scratch

_i32 = ctypes.c_int32
_p = ctypes.c_void_p


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, _i32) for n in ("kind", "n_in", "n_out", "ic", "h_in", "w_in", "oc", "k",
                                    "s", "p", "max_queue_len", "max_out_spikes")]


class QParams(ctypes.Structure):
    _fields_ = [("d_q", _p), ("q_bits", _i32), ("d_decay_table", _p), ("n_table", _i32),
                ("d_v_th", _p), ("v_th_kind", _i32), ("v_th_scalar", _i32), ("f_a", _i32),
                ("f_V", _i32), ("i_V", _i32), ("round_mode", _i32), ("overflow_mode", _i32)]


class EventsIn(ctypes.Structure):
    _fields_ = [("B", _i32), ("L", _i32), ("d_times", _p), ("d_src", _p), ("d_n_real", _p)]


class EventsOut(ctypes.Structure):
    _fields_ = [("cap", _i32), ("d_times", _p), ("d_src", _p), ("d_n", _p), ("fill_pads", _i32)]


class LayerResult(ctypes.Structure):
    _fields_ = [("d_v_final", _p), ("d_v_min", _p), ("d_v_max", _p), ("d_stats", _p)]


# Exported symbols and their ctypes signatures (include/salt_hip.h).
SIGNATURES = {
    "salt_version": ([], _i32),
    "salt_last_error": ([], ctypes.c_char_p),
    "salt_malloc": ([ctypes.POINTER(_p), ctypes.c_size_t], _i32),
    "salt_free": ([_p], _i32),
    "salt_memcpy_h2d": ([_p, _p, ctypes.c_size_t, _p], _i32),
    "salt_memcpy_d2h": ([_p, _p, ctypes.c_size_t, _p], _i32),
    "salt_stream_sync": ([_p], _i32),
    "salt_fc_transpose": ([_p, _p, _i32, _i32, _i32, _p], _i32),
    "salt_layer_workspace_size": ([ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams), _i32, _i32,
                                   _i32, ctypes.POINTER(ctypes.c_size_t)], _i32),
    "salt_layer_forward": ([ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams),
                            ctypes.POINTER(EventsIn), ctypes.POINTER(EventsOut),
                            ctypes.POINTER(LayerResult), _p, ctypes.c_size_t, _p], _i32),
    "salt_layer_forward_static": ([ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams),
                                   ctypes.POINTER(EventsIn), ctypes.POINTER(EventsOut),
                                   ctypes.POINTER(LayerResult), _p], _i32),
    "salt_stream_hash": ([_p, _p, _p, _i32, _i32, _p, _p], _i32),
    "salt_layer_trace": ([ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams),
                          ctypes.POINTER(EventsIn), _i32, _p, _p, _p, _p], _i32),
    "salt_network_workspace_size": ([_i32, ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams),
                                     _i32, _i32, _i32, ctypes.POINTER(ctypes.c_size_t)], _i32),
    "salt_network_forward": ([_i32, ctypes.POINTER(LayerDesc), ctypes.POINTER(QParams),
                              ctypes.POINTER(EventsIn), ctypes.POINTER(EventsOut),
                              ctypes.POINTER(LayerResult), _p, ctypes.c_size_t, _p], _i32),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises ImportError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                              "(spiking-affine-lazy-training_amd/csrc/build.sh)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = handle
    return _lib


class SaltError(RuntimeError):
    """A libsalt_hip.so call returned an error code."""


def check(rc: int, what: str) -> None:
    """Map C-ABI return codes to Python errors: -1 -> ValueError, others -> SaltError."""
    if rc == 0:
        return
    msg = lib().salt_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(f"{what}: {msg}")
    raise SaltError(f"{what} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def current_stream() -> int:
    return torch.cuda.current_stream().cuda_stream
