"""salt_layer_forward_static (no device allocation, static per-device scratch) against
salt_layer_forward with a caller-allocated workspace, through the C-ABI: two calls in a
row on layers whose kernels use the scratch (row-band conv with spike masks and band
lists; an FC layer sliced into spike-mask work-groups), the second call smaller than the
first, bit for bit on every output."""
import ctypes

import numpy as np
import pytest
import torch

from salt_amd import ConvLayer, FCLayer, QuantizedLayerParams, _lib
from salt_amd.quant.backend import layer_desc, prepare_params, qparams
from salt_amd.quant.codes import build_decay_table_int
from salt_amd.quant.fixed_point import RoundMode

pytestmark = pytest.mark.gpu


def _inputs(rng, B, L, n_src):
    times = np.cumsum(np.where(rng.random((B, L)) < 0.3, 0, rng.integers(1, 6, (B, L))), axis=1)
    n_real = rng.integers(L // 2, L + 1, B).astype(np.int32)
    n_real[0] = L
    times = times.astype(np.float32)
    for b in range(B):
        times[b, n_real[b]:] = 1e12
    src = rng.integers(0, n_src, (B, L)).astype(np.int32)
    dev = torch.device("cuda", 0)
    return (torch.from_numpy(times).to(dev), torch.from_numpy(src).to(dev),
            torch.from_numpy(n_real).to(dev))


def _outputs(B, N, cap):
    dev = torch.device("cuda", 0)
    return dict(t=torch.full((B, cap), -1.0, device=dev), s=torch.full((B, cap), -1, dtype=torch.int32, device=dev),
                n=torch.full((B,), -1, dtype=torch.int32, device=dev),
                v=torch.full((B, N), 7, dtype=torch.int32, device=dev),
                mn=torch.full((B, N), 7, dtype=torch.int32, device=dev),
                mx=torch.full((B, N), 7, dtype=torch.int32, device=dev),
                st=torch.full((B, 4), 7, dtype=torch.int32, device=dev))


def _call(static, layer, dp, times, src, n_real):
    lib = _lib.lib()
    B, L = times.shape
    cap = layer.max_out_spikes
    o = _outputs(B, layer.n_neurons, cap)
    desc = layer_desc(layer)
    qp = qparams(dp, RoundMode.ROUND)
    ev_in = _lib.EventsIn(B=B, L=L, d_times=times.data_ptr(), d_src=src.data_ptr(),
                          d_n_real=n_real.data_ptr())
    ev_out = _lib.EventsOut(cap=cap, d_times=o["t"].data_ptr(), d_src=o["s"].data_ptr(),
                            d_n=o["n"].data_ptr(), fill_pads=1)
    res = _lib.LayerResult(d_v_final=o["v"].data_ptr(), d_v_min=o["mn"].data_ptr(),
                           d_v_max=o["mx"].data_ptr(), d_stats=o["st"].data_ptr())
    stream = _lib.current_stream()
    if static:
        rc = lib.salt_layer_forward_static(ctypes.byref(desc), ctypes.byref(qp), ctypes.byref(ev_in),
                                           ctypes.byref(ev_out), ctypes.byref(res), stream)
        _lib.check(rc, "salt_layer_forward_static")
    else:
        ws = ctypes.c_size_t(0)
        _lib.check(lib.salt_layer_workspace_size(ctypes.byref(desc), ctypes.byref(qp), B, L, 1,
                                                 ctypes.byref(ws)), "workspace size")
        assert ws.value > 0, "the case must use a workspace"
        assert ws.value <= _lib.SALT_STATIC_SCRATCH_BYTES
        work = torch.full((ws.value,), 0xA5, dtype=torch.uint8, device=times.device)
        rc = lib.salt_layer_forward(ctypes.byref(desc), ctypes.byref(qp), ctypes.byref(ev_in),
                                    ctypes.byref(ev_out), ctypes.byref(res), work.data_ptr(),
                                    ws.value, stream)
        _lib.check(rc, "salt_layer_forward")
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in o.items()}


def _layers(rng):
    conv = ConvLayer(name="band", ic=1, h_in=130, w_in=130, oc=4, k=3, s=1, p=0, init_k=1.0,
                     max_queue_len=4000, max_out_spikes=6000)
    conv_p = QuantizedLayerParams(q=rng.integers(-127, 128, conv.weight_shape),
                                  decay_table_int=build_decay_table_int(10, 20.0), v_th_int=np.int32(90),
                                  scale=np.float32(1.0), f_a=10, f_V=0, i_V=24)
    fc = FCLayer(name="wide", n_in=64, n_out=4500, init_k=1.0, max_out_spikes=100000)
    fc_p = QuantizedLayerParams(q=rng.integers(-127, 128, fc.weight_shape),
                                decay_table_int=build_decay_table_int(10, 20.0), v_th_int=np.int32(300),
                                scale=np.float32(1.0), f_a=10, f_V=0, i_V=24)
    return [(conv, conv_p, 130 * 130, (6, 3000), (3, 1100)),
            (fc, fc_p, 64, (5, 400), (2, 150))]


@pytest.mark.parametrize("which", [0, 1])
def test_static_scratch_matches_workspace_entry_point(which):
    rng = np.random.default_rng(77 + which)
    layer, params, n_src, big, small = _layers(rng)[which]
    dp = prepare_params(layer, params, torch.device("cuda", 0))
    for shape in (big, small):  # the second call is smaller and must not see the first's data
        B, L = shape
        print("no-alloc", layer.name, "B", B, "L", L, flush=True)
        times, src, n_real = _inputs(rng, B, L, n_src)
        got = _call(True, layer, dp, times, src, n_real)
        want = _call(False, layer, dp, times, src, n_real)
        for k in want:
            np.testing.assert_array_equal(got[k], want[k], err_msg=f"{layer.name} {shape} {k}")
        assert want["n"].sum() > 0, "the case fires"


def test_static_scratch_rejects_a_layer_above_its_size():
    layer = ConvLayer(name="big", ic=2, h_in=128, w_in=128, oc=32, k=3, s=1, p=0, init_k=1.0,
                      max_queue_len=100, max_out_spikes=16)
    params = QuantizedLayerParams(q=np.ones(layer.weight_shape, np.int32),
                                  decay_table_int=build_decay_table_int(10, 20.0), v_th_int=np.int32(90),
                                  scale=np.float32(1.0), f_a=10, f_V=0, i_V=24)
    dp = prepare_params(layer, params, torch.device("cuda", 0))
    dev = torch.device("cuda", 0)
    B, L = 64, 65536
    times = torch.zeros((B, L), device=dev)
    src = torch.zeros((B, L), dtype=torch.int32, device=dev)
    n_real = torch.zeros(B, dtype=torch.int32, device=dev)
    o = _outputs(B, layer.n_neurons, 16)
    desc, qp = layer_desc(layer), qparams(dp, RoundMode.ROUND)
    ev_in = _lib.EventsIn(B=B, L=L, d_times=times.data_ptr(), d_src=src.data_ptr(), d_n_real=n_real.data_ptr())
    ev_out = _lib.EventsOut(cap=16, d_times=o["t"].data_ptr(), d_src=o["s"].data_ptr(), d_n=o["n"].data_ptr(),
                            fill_pads=1)
    res = _lib.LayerResult(d_v_final=o["v"].data_ptr(), d_v_min=None, d_v_max=None, d_stats=o["st"].data_ptr())
    rc = _lib.lib().salt_layer_forward_static(ctypes.byref(desc), ctypes.byref(qp), ctypes.byref(ev_in),
                                              ctypes.byref(ev_out), ctypes.byref(res), _lib.current_stream())
    assert rc == -1
    assert "static maximum" in _lib.lib().salt_last_error().decode()
