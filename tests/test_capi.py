"""The C-ABI library (no GPU needed): it loads, exports every symbol include/salt_hip.h
declares, and its host-side argument checks return the documented error codes."""
import ctypes
import os
import re

import pytest

from salt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "salt_hip.h"), encoding="utf-8").read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|const char\*)\s+(salt_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES)


def test_version():
    assert _lib.lib().salt_version() == 1


def _desc_fc():
    d = _lib.LayerDesc()
    d.kind, d.n_in, d.n_out, d.max_out_spikes = _lib.SALT_LAYER_FC, 8, 4, 16
    return d


def _qp(**kw):
    base = dict(d_q=1, q_bits=8, d_decay_table=1, n_table=3, d_v_th=None,
                v_th_kind=_lib.SALT_VTH_SCALAR, v_th_scalar=5, f_a=4, f_V=0, i_V=16,
                round_mode=0, overflow_mode=0)
    base.update(kw)
    return _lib.QParams(**base)


def test_workspace_size_is_host_only():
    size = ctypes.c_size_t(123)
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(_desc_fc()), ctypes.byref(_qp()), 2,
                                             10, 0, ctypes.byref(size))
    assert rc == 0 and size.value == 0  # one slice: spikes are written directly

    d = _lib.LayerDesc()
    d.kind, d.ic, d.h_in, d.w_in, d.oc, d.k, d.s, d.p = _lib.SALT_LAYER_CONV, 2, 128, 128, 32, 3, 1, 0
    d.max_queue_len, d.max_out_spikes = 100, 16
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(d), ctypes.byref(_qp()), 64, 1000, 0,
                                             ctypes.byref(size))
    assert rc == 0 and size.value == 64 * 1000 * 32 * 4  # partitioned: per-event spike masks


@pytest.mark.parametrize("kw", [dict(f_a=16), dict(i_V=31), dict(q_bits=12), dict(n_table=0),
                                dict(round_mode=3), dict(v_th_scalar=0),
                                dict(v_th_kind=_lib.SALT_VTH_PER_CHANNEL, d_v_th=None)])
def test_invalid_params_rejected(kw):
    size = ctypes.c_size_t()
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(_desc_fc()), ctypes.byref(_qp(**kw)),
                                             1, 1, 0, ctypes.byref(size))
    assert rc == -1
    assert _lib.lib().salt_last_error()


def test_unsupported_conv_geometry():
    d = _lib.LayerDesc()
    d.kind, d.ic, d.h_in, d.w_in, d.oc, d.k, d.s, d.p = _lib.SALT_LAYER_CONV, 1, 32, 32, 1, 9, 1, 0
    d.max_queue_len, d.max_out_spikes = 10, 10
    size = ctypes.c_size_t()
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(d), ctypes.byref(_qp()), 1, 1, 0,
                                             ctypes.byref(size))
    assert rc == -3 and b"candidate" in _lib.lib().salt_last_error()
