"""QuantBackend: the integer backend (salt_core/quant/backend.py:24-63) running on the GPU.

In the reference a layer builds its queue structure and hands it to backend.scan, then
extracts the spike stream itself.  Here one C-ABI call (salt_layer_forward in
libsalt_hip.so) does structure, scan and extraction event by event, so the layer hands
the backend its input stream instead (layer_forward).  scan() is kept only to say so.

Host-side checks mirror the reference's ValueErrors: non-integer codes
(quant/backend.py:14-20), shift and register widths (fixed_point.py:57-60, :79-82), mode
strings.  Three inputs the reference accepts are rejected because its results for them
depend on capacities or on JAX index clamping rather than on the model:
thresholds <= 0 (they fire on pad, catch-up and identity columns), decay codes outside
[0, 2^f_a), and source ids outside the input shape.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import NamedTuple

import numpy as np
import torch

from salt_amd import _lib
from salt_amd.capacity import LayerDiag
from salt_amd.layers.base import LayerOutput
from salt_amd.quant.fixed_point import (OverflowMode, RoundMode, check_shift_bits,
                                        check_total_bits)
from salt_amd.quant.params import QuantizedLayerParams
from salt_amd.stream import PAD_TIME, EventStream, unit_gain


class QuantLayerResult(NamedTuple):
    """One layer's integer result, the event-driven form of QuantLayerResult
    (salt_core/quant/scan.py:55-62).  The (n, queue_len) spike mask is carried by the
    output EventStream; overflowed is the any-over-steps reduction per neuron.
    Leading axis: batch."""
    v_final: torch.Tensor                # (B, n) int32 register; float32 after readout
    v_unfitted_min: torch.Tensor | None  # (B, n) int32, None when not requested
    v_unfitted_max: torch.Tensor | None  # (B, n) int32
    overflowed: torch.Tensor | None      # (B, n) bool
    spike_count: torch.Tensor            # (B,) int32
    stream_stats: torch.Tensor           # (B, 4) int32: min v_unfitted_min, max v_unfitted_max,
                                         #   needed max_queue_len (conv), overflowed (0/1)


def _check_weight_codes(q) -> None:
    """salt_core/quant/backend.py:14-20."""
    dtype = q.dtype if isinstance(q, (np.ndarray, torch.Tensor)) else np.asarray(q).dtype
    is_int = (not dtype.is_floating_point and not dtype.is_complex and dtype != torch.bool
              if isinstance(dtype, torch.dtype)
              else np.issubdtype(dtype, np.integer))
    if not is_int:
        raise ValueError(
            f"q 必須是整數權重碼(quant.codes.quantize_to_int 的 q),拿到的 dtype 是 {dtype} "
            "(q must hold integer weight codes)")


def _to_numpy(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def _as_int32(x) -> np.ndarray:
    """Integer array -> int32 with two's-complement wrap, as jnp.asarray(..., int32) does.
    An int32 array is returned as it is (no copy: weight tables can be gigabytes)."""
    a = _to_numpy(x)
    if a.dtype == np.int32:
        return a
    return a.astype(np.int64).astype(np.int32)


class DeviceLayerParams(NamedTuple):
    """Validated parameters of one layer, resident on the GPU."""
    q: torch.Tensor           # conv (oc, ic, k, k); FC transposed (n_in, n_out)
    q_bits: int
    table: torch.Tensor       # int32 decay codes
    v_th: torch.Tensor | None
    v_th_kind: int
    v_th_scalar: int
    f_a: int
    f_V: int
    i_V: int
    overflow_mode: int


def _code_bits(q: np.ndarray) -> tuple[np.ndarray, int]:
    lo, hi = (int(q.min()), int(q.max())) if q.size else (0, 0)
    if -128 <= lo and hi <= 127:
        return q.astype(np.int8), 8
    if -32768 <= lo and hi <= 32767:
        return q.astype(np.int16), 16
    return q.astype(np.int32, copy=False), 32


def prepare_params(layer, params: QuantizedLayerParams, device: torch.device) -> DeviceLayerParams:
    """Validate one layer's QuantizedLayerParams and upload them."""
    _check_weight_codes(params.q)
    f_a, f_V, i_V = int(params.f_a), int(params.f_V), int(params.i_V)
    check_shift_bits(f_a)
    if f_V < 0:
        raise ValueError(f"f_V={f_V} is negative")
    check_total_bits(i_V + f_V)
    overflow = OverflowMode(params.overflow_mode)
    q = _as_int32(params.q)
    if tuple(q.shape) != tuple(layer.weight_shape):
        raise ValueError(f"{layer.name}: q has shape {q.shape}, expected {layer.weight_shape}")
    table = _as_int32(params.decay_table_int).reshape(-1)
    if table.shape[0] < 1:
        raise ValueError(f"{layer.name}: decay_table_int is empty (delta_t_max = 0)")
    if table.min() < 0 or table.max() >= (1 << f_a):
        raise ValueError(f"{layer.name}: decay codes must lie in [0, 2^f_a) = [0, {1 << f_a}), "
                         f"got [{table.min()}, {table.max()}]")
    n = layer.n_neurons
    if params.v_th_int is None:
        v_th, kind, scalar = None, _lib.SALT_VTH_NONE, 0
    else:
        vth = np.broadcast_to(_as_int32(params.v_th_int), (n,))
        if vth.min() <= 0:
            raise ValueError(f"{layer.name}: v_th_int <= 0 is not supported (such a threshold "
                             "fires on the queue's pad, catch-up and identity columns, which "
                             "makes the reference's result depend on its capacities)")
        if (vth == vth[0]).all():
            v_th, kind, scalar = None, _lib.SALT_VTH_SCALAR, int(vth[0])
        elif hasattr(layer, "oc"):
            per_ch = vth.reshape(layer.oc, -1)
            if (per_ch == per_ch[:, :1]).all():
                v_th, kind, scalar = per_ch[:, 0].copy(), _lib.SALT_VTH_PER_CHANNEL, 0
            else:
                v_th, kind, scalar = vth.copy(), _lib.SALT_VTH_PER_NEURON, 0
        else:
            v_th, kind, scalar = vth.copy(), _lib.SALT_VTH_PER_CHANNEL, 0
    codes, bits = _code_bits(q)
    q_dev = torch.from_numpy(np.ascontiguousarray(codes)).to(device)
    if not hasattr(layer, "oc"):  # FC: transpose once to (n_in, n_out) on the device
        q_t = torch.empty((layer.n_in, layer.n_out), dtype=q_dev.dtype, device=device)
        _lib.check(_lib.lib().salt_fc_transpose(q_dev.data_ptr(), q_t.data_ptr(), layer.n_out,
                                                layer.n_in, bits, _lib.current_stream()),
                   "salt_fc_transpose")
        q_dev = q_t
    return DeviceLayerParams(
        q=q_dev, q_bits=bits, table=torch.from_numpy(table.copy()).to(device),
        v_th=None if v_th is None else torch.from_numpy(np.ascontiguousarray(v_th)).to(device),
        v_th_kind=kind, v_th_scalar=scalar, f_a=f_a, f_V=f_V, i_V=i_V,
        overflow_mode=_lib.SALT_SATURATE if overflow is OverflowMode.SATURATE else _lib.SALT_WRAP)


def layer_desc(layer) -> _lib.LayerDesc:
    d = _lib.LayerDesc()
    if hasattr(layer, "oc"):
        d.kind = _lib.SALT_LAYER_CONV
        d.ic, d.h_in, d.w_in = layer.ic, layer.h_in, layer.w_in
        d.oc, d.k, d.s, d.p = layer.oc, layer.k, layer.s, layer.p
        d.max_queue_len = layer.max_queue_len
    else:
        d.kind = _lib.SALT_LAYER_FC
        d.n_in, d.n_out = layer.n_in, layer.n_out
    d.max_out_spikes = layer.max_out_spikes
    return d


def qparams(dp: DeviceLayerParams, round_mode: RoundMode) -> _lib.QParams:
    return _lib.QParams(
        d_q=dp.q.data_ptr(), q_bits=dp.q_bits, d_decay_table=dp.table.data_ptr(),
        n_table=dp.table.shape[0], d_v_th=None if dp.v_th is None else dp.v_th.data_ptr(),
        v_th_kind=dp.v_th_kind, v_th_scalar=dp.v_th_scalar, f_a=dp.f_a, f_V=dp.f_V, i_V=dp.i_V,
        round_mode=_lib.SALT_TRUNCATE if round_mode is RoundMode.TRUNCATE else _lib.SALT_ROUND,
        overflow_mode=dp.overflow_mode)


class RawLayerOut(NamedTuple):
    times: torch.Tensor
    src: torch.Tensor
    n: torch.Tensor
    v_final: torch.Tensor
    v_min: torch.Tensor | None
    v_max: torch.Tensor | None
    stats: torch.Tensor


def run_layer_kernel(layer, dp: DeviceLayerParams, round_mode: RoundMode, times: torch.Tensor,
                     src: torch.Tensor, n_real: torch.Tensor, cap: int, *, extremes: bool,
                     fill_pads: bool) -> RawLayerOut:
    """One salt_layer_forward call over batched device tensors (B, L)."""
    lib = _lib.lib()
    dev = times.device
    B, L = times.shape
    n = layer.n_neurons
    desc = layer_desc(layer)
    desc.max_out_spikes = cap
    qp = qparams(dp, round_mode)
    ws = ctypes.c_size_t(0)
    _lib.check(lib.salt_layer_workspace_size(ctypes.byref(desc), ctypes.byref(qp), B, L,
                                             int(extremes), ctypes.byref(ws)),
               "salt_layer_workspace_size")
    workspace = torch.empty(max(ws.value, 1), dtype=torch.uint8, device=dev)
    out = RawLayerOut(
        times=torch.empty((B, cap), dtype=torch.float32, device=dev),
        src=torch.empty((B, cap), dtype=torch.int32, device=dev),
        n=torch.empty(B, dtype=torch.int32, device=dev),
        v_final=torch.empty((B, n), dtype=torch.int32, device=dev),
        v_min=torch.empty((B, n), dtype=torch.int32, device=dev) if extremes else None,
        v_max=torch.empty((B, n), dtype=torch.int32, device=dev) if extremes else None,
        stats=torch.empty((B, 4), dtype=torch.int32, device=dev))
    ev_in = _lib.EventsIn(B=B, L=L, d_times=times.data_ptr(), d_src=src.data_ptr(),
                          d_n_real=n_real.data_ptr())
    ev_out = _lib.EventsOut(cap=cap, d_times=out.times.data_ptr(), d_src=out.src.data_ptr(),
                            d_n=out.n.data_ptr(), fill_pads=int(fill_pads))
    res = _lib.LayerResult(d_v_final=out.v_final.data_ptr(), d_v_min=_lib.ptr(out.v_min),
                           d_v_max=_lib.ptr(out.v_max), d_stats=out.stats.data_ptr())
    _lib.check(lib.salt_layer_forward(ctypes.byref(desc), ctypes.byref(qp), ctypes.byref(ev_in),
                                      ctypes.byref(ev_out), ctypes.byref(res),
                                      workspace.data_ptr(), ws.value, _lib.current_stream()),
               f"salt_layer_forward({layer.name})")
    return out


def reference_truncation(times: np.ndarray, src: np.ndarray, n: np.ndarray, cap: int,
                         n_neurons: int) -> tuple[np.ndarray, np.ndarray]:
    """Streams whose spike count exceeds cap, as salt_core/stream.py:49-64 cuts them: keep
    the first cap spikes in (neuron, column) order, then order them by event.
    times/src: full streams (B, >= max n) in (event, neuron) order."""
    B = times.shape[0]
    out_t = np.full((B, cap), np.float32(PAD_TIME), np.float32)
    out_s = np.zeros((B, cap), np.int32)
    for b in range(B):
        nb = int(n[b])
        if nb <= cap:
            out_t[b, :nb], out_s[b, :nb] = times[b, :nb], src[b, :nb]
            continue
        s = src[b, :nb].astype(np.int64)
        counts = np.bincount(s, minlength=n_neurons)
        start = np.concatenate([[0], np.cumsum(counts)[:-1]])
        order = np.argsort(s, kind="stable")             # neuron-major, event order inside
        rank = np.empty(nb, np.int64)
        rank[order] = np.arange(nb) - start[s[order]]    # rank of a spike within its neuron
        keep = (start[s] + rank) < cap
        out_t[b], out_s[b] = times[b, :nb][keep], src[b, :nb][keep]
    return out_t, out_s


def _batched(t: torch.Tensor) -> torch.Tensor:
    return t if t.dim() == 2 else t.unsqueeze(0)


@dataclass(frozen=True)
class QuantBackend:
    """Integer backend (salt_core/quant/backend.py:24-63).

    round_mode: rounding after the decay multiply, shared by the whole network.
    neuron_extremes: compute v_unfitted_min/max per neuron (QuantLayerResult fields); the
        per-stream reductions the reference's driver reports are always computed.
    """
    round_mode: RoundMode | str = RoundMode.ROUND
    neuron_extremes: bool = True

    def scan(self, *args, **kwargs):
        raise NotImplementedError(
            "the GPU integer path does not build queue structures: layers call "
            "QuantBackend.layer_forward with their input stream instead")

    def readout(self, result: QuantLayerResult, params: QuantizedLayerParams) -> QuantLayerResult:
        """v_final -> v_int * 2^-f_V * s_c per neuron, float32 (salt_core/quant/backend.py:55-63)."""
        scale = torch.as_tensor(_to_numpy(params.scale).astype(np.float32),
                                device=result.v_final.device)
        v = result.v_final.to(torch.float32) * np.float32(2.0 ** -params.f_V) * scale
        return result._replace(v_final=v)

    # -------------------------------------------------------------- device path

    def device_params(self, layer, params: QuantizedLayerParams,
                      device: torch.device) -> DeviceLayerParams:
        """Validated, uploaded parameters, cached per (params object, layer)."""
        key = (id(params), layer.weight_shape, getattr(layer, "name", None), str(device))
        hit = _PARAM_CACHE.get(key)
        if hit is not None and hit[0] is params:
            return hit[1]
        dp = prepare_params(layer, params, device)
        if len(_PARAM_CACHE) > 64:
            _PARAM_CACHE.clear()
        _PARAM_CACHE[key] = (params, dp)  # keeps params alive, so its id stays unique
        return dp

    def layer_forward(self, layer, params: QuantizedLayerParams, in_stream: EventStream, *,
                      fill_pads: bool = True, exact_truncation: bool = True) -> LayerOutput:
        """One layer over a (batched) EventStream on the GPU: the work of
        ConvLayer.forward / FCLayer.forward (salt_core/layers/conv.py:124-149,
        salt_core/layers/fc.py:84-101) under this backend.

        exact_truncation=False: no host synchronisation; a stream with more spikes than
        the layer's capacity keeps its first cap spikes in event order, not the
        reference's choice (the first cap in (neuron, column) order) -- for callers that
        check the counts afterwards and redo such a layer (run_network does)."""
        round_mode = RoundMode(self.round_mode)
        single = in_stream.event_times.dim() == 1
        times = _batched(in_stream.event_times).to(torch.float32).contiguous()
        src = _batched(in_stream.event_source_idx).to(torch.int32).contiguous()
        n_real = in_stream.n_real_events.reshape(-1).to(torch.int32).contiguous()
        if not times.is_cuda:
            raise ValueError("the event stream must live on the GPU")
        dp = self.device_params(layer, params, times.device)
        cap = int(layer.max_out_spikes)
        raw = run_layer_kernel(layer, dp, round_mode, times, src, n_real, cap,
                               extremes=self.neuron_extremes, fill_pads=fill_pads)
        out_t, out_s = raw.times, raw.src
        n_host = raw.n.cpu().numpy() if exact_truncation else None
        if exact_truncation and (n_host > cap).any():
            # Rerun with room for every spike, then cut as the reference does.
            full = run_layer_kernel(layer, dp, round_mode, times, src, n_real, int(n_host.max()),
                                    extremes=False, fill_pads=False)
            t_sel, s_sel = reference_truncation(full.times.cpu().numpy(), full.src.cpu().numpy(),
                                                n_host, cap, layer.n_neurons)
            out_t = torch.from_numpy(t_sel).to(times.device)
            out_s = torch.from_numpy(s_sel).to(times.device)
        overflowed = None
        if raw.v_min is not None:
            half = 1 << (dp.i_V + dp.f_V - 1)
            overflowed = (raw.v_min < -half) | (raw.v_max > half - 1)
        result = QuantLayerResult(v_final=raw.v_final, v_unfitted_min=raw.v_min,
                                  v_unfitted_max=raw.v_max, overflowed=overflowed,
                                  spike_count=raw.n, stream_stats=raw.stats)
        needed = {"max_out_spikes": raw.n, "max_extra_steps": torch.zeros_like(raw.n)}
        if hasattr(layer, "oc"):
            needed = {"max_queue_len": raw.stats[:, 2], **needed}
        firing = raw.n.to(torch.float32) / (layer.n_neurons * n_real.clamp(min=1).to(torch.float32))
        diag = LayerDiag(spike_count=raw.n, firing_rate=firing, needed=needed)
        stream = EventStream(event_times=out_t, event_source_idx=out_s,
                             event_gain=unit_gain(out_t), n_real_events=raw.n)
        if single:
            stream = EventStream(*(x[0] for x in stream))
            result = QuantLayerResult(*(None if x is None else x[0] for x in result))
            diag = LayerDiag(diag.spike_count[0], diag.firing_rate[0],
                             {k: v[0] for k, v in diag.needed.items()})
        return LayerOutput(stream=stream, result=result, diag=diag, trace=None)


    def layer_trace(self, layer, params: QuantizedLayerParams, in_stream: EventStream):
        """The layer's step-by-step trajectories over a (batched) EventStream
        (salt_core/quant/scan.py:83-95 under trace=True): salt_layer_trace."""
        from salt_amd.trace import LayerForwardTrace
        round_mode = RoundMode(self.round_mode)
        single = in_stream.event_times.dim() == 1
        times = _batched(in_stream.event_times).to(torch.float32).contiguous()
        src = _batched(in_stream.event_source_idx).to(torch.int32).contiguous()
        n_real = in_stream.n_real_events.reshape(-1).to(torch.int32).contiguous()
        if not times.is_cuda:
            raise ValueError("the event stream must live on the GPU")
        dp = self.device_params(layer, params, times.device)
        B, L = times.shape
        steps = int(layer.max_queue_len) if hasattr(layer, "oc") else L
        n = layer.n_neurons
        v_steps = torch.empty((B, n, steps), dtype=torch.int32, device=times.device)
        event_ms = torch.empty((B, n, steps), dtype=torch.float32, device=times.device)
        flags = torch.empty((B, n, steps), dtype=torch.uint8, device=times.device)
        desc = layer_desc(layer)
        qp = qparams(dp, round_mode)
        ev_in = _lib.EventsIn(B=B, L=L, d_times=times.data_ptr(), d_src=src.data_ptr(),
                              d_n_real=n_real.data_ptr())
        _lib.check(_lib.lib().salt_layer_trace(ctypes.byref(desc), ctypes.byref(qp),
                                               ctypes.byref(ev_in), steps, v_steps.data_ptr(),
                                               event_ms.data_ptr(), flags.data_ptr(),
                                               _lib.current_stream()),
                   f"salt_layer_trace({layer.name})")
        tr = LayerForwardTrace(spike_mask=(flags & 1).bool(), v_steps=v_steps,
                               event_ms=event_ms, overflowed=(flags & 2).bool())
        if single:
            tr = LayerForwardTrace(*(x[0] for x in tr))
        return tr


_PARAM_CACHE: dict = {}
QUANT = QuantBackend()


def resolve_backend(backend) -> QuantBackend:
    """Layers run only on the integer backend; None means the default QuantBackend()."""
    if backend is None:
        return QUANT
    if not isinstance(backend, QuantBackend):
        raise ValueError(f"only QuantBackend is supported on this path, got {type(backend).__name__}")
    return backend
