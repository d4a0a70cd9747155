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


def test_workspace_size_is_host_only(monkeypatch):
    size = ctypes.c_size_t(123)
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(_desc_fc()), ctypes.byref(_qp()), 2,
                                             10, 0, ctypes.byref(size))
    assert rc == 0 and size.value == 0  # one slice: spikes are written directly

    d = _lib.LayerDesc()
    d.kind, d.ic, d.h_in, d.w_in, d.oc, d.k, d.s, d.p = _lib.SALT_LAYER_CONV, 2, 128, 128, 32, 3, 1, 0
    d.max_queue_len, d.max_out_spikes = 100, 16
    # partitioned (row bands of >= 2 rows, 5 channel groups of one iteration): a validity
    # word per event, the spike words of the 2 bands an event reaches at most (one 8-byte
    # word per channel group), one spike count per (stream, 2048-event compaction
    # segment), then (unless turned off) each band's event list
    masks_and_counts = 64 * 1000 * 4 + 64 * 1000 * 2 * 5 * 8 + 64 * 1 * 4
    monkeypatch.setenv("SALT_CONV_BANDLIST", "0")
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(d), ctypes.byref(_qp()), 64, 1000, 0,
                                             ctypes.byref(size))
    assert rc == 0 and size.value == masks_and_counts
    monkeypatch.delenv("SALT_CONV_BANDLIST")
    rc = _lib.lib().salt_layer_workspace_size(ctypes.byref(d), ctypes.byref(_qp()), 64, 1000, 0,
                                             ctypes.byref(size))
    assert rc == 0 and size.value > masks_and_counts + 64 * 1000 * 4


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


def _chain(fc_n_out=4):
    """conv 2x128x128 -> 32 3x3 s1 (partitioned: per-event spike masks) -> FC."""
    d = (_lib.LayerDesc * 2)()
    d[0].kind, d[0].ic, d[0].h_in, d[0].w_in, d[0].oc, d[0].k, d[0].s, d[0].p = 1, 2, 128, 128, 32, 3, 1, 0
    d[0].max_queue_len, d[0].max_out_spikes = 100, 5000
    d[1].kind, d[1].n_in, d[1].n_out, d[1].max_out_spikes = 0, 32 * 126 * 126, fc_n_out, 64
    q = (_lib.QParams * 2)(_qp(), _qp())
    return d, q


@pytest.mark.parametrize("fc_n_out", [4, 5000])
def test_network_workspace_is_the_largest_layer_workspace(fc_n_out):
    d, q = _chain(fc_n_out)
    lib = _lib.lib()
    sizes = []
    for i, L in enumerate((1000, d[0].max_out_spikes)):  # layer 1 reads layer 0's stream
        s = ctypes.c_size_t()
        assert lib.salt_layer_workspace_size(ctypes.byref(d[i]), ctypes.byref(q[i]), 64, L, 0,
                                             ctypes.byref(s)) == 0
        sizes.append(s.value)
    size = ctypes.c_size_t()
    assert lib.salt_network_workspace_size(2, d, q, 64, 1000, 0, ctypes.byref(size)) == 0
    assert size.value == max(sizes) > 0
    # beyond 4 waves x 1024 neurons per stream, FC slices write spike masks too
    assert (sizes[1] > 0) == (fc_n_out > 4096)


def test_network_rejects_mismatched_chain():
    d, q = _chain()
    d[1].n_in -= 1
    size = ctypes.c_size_t()
    assert _lib.lib().salt_network_workspace_size(2, d, q, 1, 1, 0, ctypes.byref(size)) == -1
    assert b"layer 1 takes" in _lib.lib().salt_last_error()


def test_network_checks_every_layer_before_launching():
    """A bad parameter in the last layer fails the call before the first layer is
    enqueued (no device is touched: the pointers here are placeholders)."""
    d, q = _chain()
    q[1] = _qp(f_a=16)
    ev_in = _lib.EventsIn(B=2, L=10, d_times=8, d_src=8, d_n_real=8)
    outs = (_lib.EventsOut * 2)(*[_lib.EventsOut(cap=d[i].max_out_spikes, d_times=8, d_src=8,
                                                 d_n=8, fill_pads=0) for i in range(2)])
    res = (_lib.LayerResult * 2)(*[_lib.LayerResult(d_v_final=8, d_v_min=None, d_v_max=None,
                                                    d_stats=8) for _ in range(2)])
    rc = _lib.lib().salt_network_forward(2, d, q, ctypes.byref(ev_in), outs, res, 8, 1 << 40,
                                         None)
    assert rc == -1 and b"MAX_SHIFT_BITS" in _lib.lib().salt_last_error()


def test_probe_library_exports_its_header():
    """libsalt_probe.so (bench.py's LDS probe) exports what include/salt_probe.h declares."""
    text = open(os.path.join(ROOT, "include", "salt_probe.h"), encoding="utf-8").read()
    names = re.findall(r"^\s*int32_t\s+(salt_\w+)\s*\(", text, re.M)
    assert names == ["salt_probe_lds"]
    probe = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libsalt_probe.so"))
    for name in names:
        assert hasattr(probe, name), name
