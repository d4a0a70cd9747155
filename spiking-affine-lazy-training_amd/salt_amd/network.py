"""Network container: InputEvents, Network and run_network with the API of
salt_core/network.py.  Every layer runs on the GPU integer path (QuantBackend).

apply() takes one sample (arrays without a batch axis), apply_batched() a batch; both
issue one batched launch per layer.  Host arrays are validated as InputEvents.checked
does and uploaded; device tensors are used as given (like the reference's jit path,
which cannot check either).
"""
from __future__ import annotations

import math
from collections import Counter
from collections.abc import Sequence
from dataclasses import dataclass, replace
from typing import Any, NamedTuple

import numpy as np
import torch

from salt_amd.quant.backend import QuantBackend, resolve_backend
from salt_amd.stream import EventStream, unit_gain

_MAX_EVENT_TIME = 2 ** 31  # salt_core/network.py:23


class InputEvents(NamedTuple):
    """Network input (salt_core/network.py:26-54): integer-ms times, flat source ids over
    the input shape, number of real events; optional leading batch axis."""
    event_times: Any
    source_idx: Any
    n_real_events: Any

    @staticmethod
    def checked(event_times, source_idx, n_real_events) -> "InputEvents":
        """Host check of the real events' times (salt_core/network.py:34-54): integer,
        in [0, 2^31), non-decreasing; pads are not checked.  Raises ValueError."""
        times = _host(event_times)
        n_real = _host(n_real_events)
        is_real = np.arange(times.shape[-1]) < n_real[..., None]
        real_times = times[is_real]
        if not np.all(real_times == np.floor(real_times)):
            raise ValueError("事件時間必須是整數毫秒 (event times must be integer ms)")
        # The range is also checked on the float32 values the kernels receive: float64
        # times in [2^31 - 64, 2^31) round up to 2^31 there.
        if (np.any(real_times < 0) or np.any(real_times >= _MAX_EVENT_TIME)
                or np.any(real_times.astype(np.float32) >= np.float32(_MAX_EVENT_TIME))):
            raise ValueError(f"事件時間必須在 [0, 2^31) 裡,拿到的範圍是 "
                             f"[{real_times.min()}, {real_times.max()}]")
        both_real = is_real[..., 1:]
        if np.any(np.diff(times, axis=-1)[both_real] < 0):
            raise ValueError("真事件時間必須不遞減 (real event times must be non-decreasing)")
        return InputEvents(event_times=event_times, source_idx=source_idx,
                           n_real_events=n_real_events)


def _host(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


class NetworkOutput(NamedTuple):
    """run_network's output (salt_core/network.py:57-67)."""
    results: tuple
    diags: tuple
    traces: tuple | None  # LayerForwardTrace per layer when run with trace=True
    fits: torch.Tensor  # bool: every layer with a capacity held this input

    @property
    def last(self):
        return self.results[-1]


def _check_connected(out_shape, in_shape, out_name: str, in_name: str) -> None:
    """salt_core/network.py:70-84."""
    out_shape, in_shape = tuple(out_shape), tuple(in_shape)
    connected = math.prod(out_shape) == in_shape[0] if len(in_shape) == 1 else out_shape == in_shape
    if connected:
        return
    if len(out_shape) < len(in_shape):
        raise ValueError(f"{out_name} 的輸出 {out_shape} 沒有空間形狀,"
                         f"不能接吃空間輸入的 {in_name}(輸入 {in_shape})")
    raise ValueError(f"{out_name} 的輸出 {out_shape} 接不上 {in_name} 的輸入 {in_shape}")


def check_layer_connections(layers: Sequence) -> None:
    for prev, nxt in zip(layers, layers[1:]):
        _check_connected(prev.output_shape, nxt.input_shape, prev.name, nxt.name)


def _chain(layers: Sequence, weights: Sequence, input_stream: EventStream, backend) -> list:
    """The layers' outputs, enqueued one after the other with no host synchronisation in
    between, then one check of every layer's spike counts against its capacity.  Only
    when a stream overflowed a layer's capacity is that layer (and every layer after it)
    run again with the reference's truncation, which needs the counts on the host."""
    outputs, stream = [], input_stream
    for layer, params in zip(layers, weights):
        out = backend.layer_forward(layer, params, stream, exact_truncation=False)
        outputs.append(out)
        stream = out.stream
    over = torch.stack([(o.diag.spike_count.reshape(-1) > int(layer.max_out_spikes)).any()
                        for layer, o in zip(layers, outputs)]).cpu().numpy()
    if not over.any():
        return outputs
    first = int(np.flatnonzero(over)[0])
    stream = outputs[first - 1].stream if first else input_stream
    for i in range(first, len(layers)):
        outputs[i] = layers[i].forward(weights[i], stream, backend=backend)
        stream = outputs[i].stream
    return outputs


def run_network(layers: Sequence, weights: Sequence, input_stream: EventStream, *,
                backend: QuantBackend | None = None, trace: bool = False) -> NetworkOutput:
    """Chain layers, each output stream feeding the next (salt_core/network.py:93-122).
    trace: also collect every layer's step-by-step trajectories (LayerForwardTrace)."""
    backend = resolve_backend(backend)
    check_layer_connections(layers)
    outputs = _chain(layers, weights, input_stream, backend) if not trace else []
    if trace:
        stream = input_stream
        for layer, params in zip(layers, weights):
            out = layer.forward(params, stream, backend=backend, trace=True)
            outputs.append(out)
            stream = out.stream
    fits = None
    for layer, out in zip(layers, outputs):
        if layer.capacity is not None:
            f = layer.capacity.fits(out.diag)
            fits = f if fits is None else fits & f
    return NetworkOutput(results=tuple(o.result for o in outputs),
                         diags=tuple(o.diag for o in outputs),
                         traces=tuple(o.trace for o in outputs) if trace else None, fits=fits)


@dataclass(frozen=True)
class Network:
    """input_shape plus a list of layers (salt_core/network.py:125-187)."""
    input_shape: tuple[int, ...]
    layers: tuple

    def __post_init__(self) -> None:
        object.__setattr__(self, "input_shape", tuple(int(v) for v in self.input_shape))
        object.__setattr__(self, "layers", tuple(self.layers))
        if not self.layers:
            raise ValueError("layers 不能是空的")
        _check_connected(self.input_shape, self.layers[0].input_shape, "輸入", self.layers[0].name)
        check_layer_connections(self.layers)

    @classmethod
    def build(cls, input_shape: Sequence[int], specs: Sequence) -> "Network":
        """Connect layer specs, naming unnamed ones conv1, conv2, fc1, ...
        (salt_core/network.py:143-158)."""
        shape = tuple(int(v) for v in input_shape)
        counts: Counter[str] = Counter()
        layers = []
        for spec in specs:
            counts[spec.name_prefix] += 1
            layer = spec.build(shape, spec.name or f"{spec.name_prefix}{counts[spec.name_prefix]}")
            layers.append(layer)
            shape = layer.output_shape
        return cls(input_shape=input_shape, layers=layers)

    def input_stream(self, raw: InputEvents, device: torch.device | None = None) -> EventStream:
        """Raw input -> first layer's stream: times as float32 (the reference holds them
        as float32 too), source ids copied as int32, gain 1 (salt_core/network.py:165-171).
        Host arrays are checked (times, and source ids within the input shape) and
        uploaded."""
        device = device or torch.device("cuda", torch.cuda.current_device())
        t, s, n = raw
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            InputEvents.checked(t, s, n)
            src = _host(s)
            n_real = _host(n)
            is_real = np.arange(src.shape[-1]) < n_real[..., None]
            n_src = math.prod(self.input_shape)
            bad = (src < 0) | (src >= n_src)
            if np.any(bad & is_real):
                raise ValueError(f"source_idx must lie in [0, {n_src}) for every real event")
            t = torch.from_numpy(np.ascontiguousarray(_host(t), dtype=np.float32)).to(device)
            s = torch.from_numpy(np.ascontiguousarray(src.astype(np.int64).astype(np.int32))).to(device)
            n = torch.from_numpy(np.ascontiguousarray(n_real, dtype=np.int32)).to(device)
        t = t.to(torch.float32)
        return EventStream(event_times=t, event_source_idx=s.to(torch.int32),
                           event_gain=unit_gain(t), n_real_events=torch.as_tensor(n).to(torch.int32))

    def apply(self, weights: Sequence, raw: InputEvents, *, backend: QuantBackend | None = None,
              trace: bool = False) -> NetworkOutput:
        """One sample (salt_core/network.py:173-177)."""
        return run_network(self.layers, weights, self.input_stream(raw), backend=backend,
                           trace=trace)

    def apply_batched(self, weights: Sequence, raw_batch: InputEvents, *,
                      backend: QuantBackend | None = None, trace: bool = False) -> NetworkOutput:
        """A batch with shared weights (salt_core/network.py:179-183): one launch per layer."""
        return run_network(self.layers, weights, self.input_stream(raw_batch), backend=backend,
                           trace=trace)

    def replace_layers(self, layers: Sequence) -> "Network":
        return replace(self, layers=tuple(layers))
