"""Running a quantized model over many samples: quant_forward_split, run_until_fits and
the per-sample reference fields (example/quant_run.py:54-132).

Also the overflow analysis of a run (headroom, fewest extra register bits;
example/quant_run.py:139-240).

Each batch is one NetworkRunner.run (every layer on the GPU, no host synchronisation
between layers).  When a stream of a batch overflowed the output capacity of a layer
that feeds another, that batch is run again layer by layer through
Network.apply_batched, which cuts the stream as the reference does before the next layer
sees it, so every field equals the reference's for every sample.
"""
from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np
import torch

from salt_amd.capacity import LayerDiag, grown_to_fit
from salt_amd.data.events import take_input_events
from salt_amd.network import InputEvents, Network
from salt_amd.quant.backend import QuantBackend
from salt_amd.quant.fixed_point import OverflowMode, RoundMode
from salt_amd.runner import NetworkRunner


class QuantSplitOutput(NamedTuple):
    """example/quant_run.py:54-63; N = number of samples."""
    v_final_int: np.ndarray     # (N, n_out) int32 output-layer registers
    preds: np.ndarray           # (N,) int32
    spike_count: np.ndarray     # (N, n_layers) int32
    truncated: np.ndarray       # (N, n_layers) bool, a capacity exceeded
    overflowed: np.ndarray      # (N, n_layers) bool, a register overflowed
    v_unfitted_min: np.ndarray  # (N, n_layers) int32, min pre-write-back value over neurons
    v_unfitted_max: np.ndarray  # (N, n_layers) int32
    needed: dict                # layer name -> knob -> (N,) needed capacity


REFERENCE_FIELDS = ("v_final_int", "preds", "spike_count", "truncated", "overflowed")
_ARRAY_FIELDS = REFERENCE_FIELDS + ("v_unfitted_min", "v_unfitted_max")


def _batches(raw: InputEvents, batch_size: int):
    n = np.asarray(raw.event_times).shape[0]
    for start in range(0, n, batch_size):
        yield take_input_events(raw, slice(start, start + batch_size))


def readout_scores(v_final: torch.Tensor, params) -> np.ndarray:
    """QuantBackend.readout then membrane-regression decode: float32
    v_int * 2^-f_V * s_c per neuron (salt_core/quant/backend.py:55-63)."""
    scale = torch.as_tensor(np.asarray(params.scale, dtype=np.float32), device=v_final.device)
    return (v_final.to(torch.float32) * np.float32(2.0 ** -int(params.f_V)) * scale).cpu().numpy()


class _Readout(NamedTuple):
    """The last layer's result after readout, as the decoder reads it."""
    v_final: np.ndarray


def _layer_needed(layer, n: torch.Tensor, stats: torch.Tensor) -> dict:
    """The knobs of layers/conv.py:137-141 and layers/fc.py:92-94 (the integer backend
    needs no extra scan steps)."""
    needed = {"max_out_spikes": n, "max_extra_steps": torch.zeros_like(n)}
    if hasattr(layer, "oc"):
        needed = {"max_queue_len": stats[:, 2], **needed}
    return needed


def _run_batch(network: Network, runner: NetworkRunner, backend: QuantBackend, params,
               decoder, batch: InputEvents, device) -> dict:
    stream = network.input_stream(batch, device=device)
    outs = runner.run(stream)
    layers = network.layers
    overfull = any(bool((o.n > l.max_out_spikes).any()) for o, l in zip(outs[:-1], layers[:-1]))
    if overfull:
        res = network.apply_batched(params, batch, backend=backend).results
        ns = [r.spike_count for r in res]
        stats = [r.stream_stats for r in res]
        v_last = res[-1].v_final
    else:
        ns = [o.n for o in outs]
        stats = [o.stats for o in outs]
        v_last = outs[-1].v_final
    scores, _ = decoder.decode(_Readout(readout_scores(v_last, params[-1])))
    truncated, needed = [], []
    for layer, n, st in zip(layers, ns, stats):
        nd = _layer_needed(layer, n, st)
        needed.append({k: v.cpu().numpy() for k, v in nd.items()})
        if layer.capacity is None:
            truncated.append(np.zeros(n.shape[0], bool))
        else:
            diag = LayerDiag(spike_count=n, firing_rate=torch.zeros_like(n, dtype=torch.float32),
                             needed=nd)
            truncated.append(~layer.capacity.fits(diag).cpu().numpy())
    return {"v_final_int": v_last.cpu().numpy(),
            "preds": np.argmax(scores, axis=1).astype(np.int32),
            "spike_count": np.stack([n.cpu().numpy() for n in ns], axis=1),
            "truncated": np.stack(truncated, axis=1),
            "overflowed": np.stack([st[:, 3].cpu().numpy() != 0 for st in stats], axis=1),
            "v_unfitted_min": np.stack([st[:, 0].cpu().numpy() for st in stats], axis=1),
            "v_unfitted_max": np.stack([st[:, 1].cpu().numpy() for st in stats], axis=1),
            "needed": needed}


def quant_forward_split(network: Network, decoder, params, round_mode: RoundMode | str,
                        raw: InputEvents, batch_size: int, *, device=None) -> QuantSplitOutput:
    """Every sample of raw through the integer network in batches of batch_size
    (example/quant_run.py:71-103)."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    runner = NetworkRunner(network, params, round_mode, device)
    backend = QuantBackend(round_mode=round_mode, neuron_extremes=False)
    parts = [_run_batch(network, runner, backend, params, decoder, b, device)
             for b in _batches(raw, batch_size)]
    arrays = {k: np.concatenate([p[k] for p in parts]) for k in _ARRAY_FIELDS}
    needed = {layer.name: {knob: np.concatenate([p["needed"][i][knob] for p in parts])
                           for knob in parts[0]["needed"][i]}
              for i, layer in enumerate(network.layers)}
    return QuantSplitOutput(**arrays, needed=needed)


def reference_arrays(out: QuantSplitOutput) -> dict[str, np.ndarray]:
    """The per-sample fields stored in reference.npz (example/quant_run.py:106-108)."""
    return {key: getattr(out, key) for key in REFERENCE_FIELDS}


def grown_for_needed(layers, policies: dict, needed: dict) -> list:
    """Each layer grown for the largest need over all samples
    (example/quant_run.py:111-119)."""
    diags = [LayerDiag(spike_count=0, firing_rate=0.0,
                       needed={k: int(np.max(v)) for k, v in needed[layer.name].items()})
             for layer in layers]
    return grown_to_fit(layers, policies, diags)


def run_until_fits(network: Network, decoder, params, round_mode: RoundMode | str,
                   raw: InputEvents, batch_size: int, policies: dict, *, device=None
                   ) -> tuple[Network, QuantSplitOutput, int]:
    """quant_forward_split, growing the capacities and running again while any sample
    is truncated; returns (network that fits, output, number of regrows)
    (example/quant_run.py:122-132)."""
    n_regrow = 0
    out = quant_forward_split(network, decoder, params, round_mode, raw, batch_size, device=device)
    while out.truncated.any():
        network = network.replace_layers(grown_for_needed(network.layers, policies, out.needed))
        out = quant_forward_split(network, decoder, params, round_mode, raw, batch_size,
                                  device=device)
        n_regrow += 1
    return network, out, n_regrow


def headroom_bits(params, out) -> list:
    """Per layer, bits between the largest pre-write-back magnitude and the register's
    range, (w - 1) - log2(max(-min, max + 1)); None when the layer stayed at 0
    (example/quant_run.py:144-156)."""
    result = []
    for i, p in enumerate(params):
        peak = max(-int(out.v_unfitted_min[:, i].min()), int(out.v_unfitted_max[:, i].max()) + 1)
        result.append(None if peak <= 0 else round(p.i_V + p.f_V - 1 - math.log2(peak), 3))
    return result


def with_extra_i_V(params, extra: list[int]) -> list:
    """example/quant_run.py:139-141."""
    return [p._replace(i_V=p.i_V + e) for p, e in zip(params, extra)]


def min_extra_bits(network, decoder, params, round_mode, raw, batch_size: int, policies: dict,
                   out, *, device=None) -> tuple[list[int], int]:
    """Adds one bit to the most upstream overflowing layer and re-runs until no sample
    overflows (example/quant_run.py:159-177).  Returns (bits per layer, rounds)."""
    extra = [0] * len(params)
    rounds = 0
    while out.overflowed.any():
        extra[int(np.argmax(out.overflowed.any(axis=0)))] += 1
        _, out, _ = run_until_fits(network, decoder, with_extra_i_V(params, extra), round_mode,
                                   raw, batch_size, policies, device=device)
        rounds += 1
    return extra, rounds


MAX_OVERFLOW_EVENTS = 50  # example/quant_run.py:20-21


def _neuron_position(layer, neuron: int) -> tuple[int, int, int]:
    """Neuron id -> (channel, y, x); FC neurons are (neuron, 0, 0)."""
    shape = (layer.oc, layer.h_out, layer.w_out) if hasattr(layer, "oc") else (layer.n_out, 1, 1)
    return tuple(int(v) for v in np.unravel_index(neuron, shape))


def overflow_events(network: Network, params, round_mode: RoundMode | str, raw: InputEvents,
                    out: QuantSplitOutput) -> list[dict]:
    """Where registers overflowed: for every overflowing (sample, layer, neuron), its
    first overflowing step, from a traced re-run of that sample
    (example/quant_run.py:180-210).  At most MAX_OVERFLOW_EVENTS entries.  v_before /
    v_after: the register before and after that step (0 after a spike); true_min /
    true_max: the neuron's extremes of the value before write-back over the sample."""
    backend = QuantBackend(round_mode=round_mode)
    events = []
    for i in np.nonzero(out.overflowed.any(axis=1))[0]:
        one = InputEvents(*(np.asarray(a)[int(i)] for a in raw))
        output = network.apply(params, one, backend=backend, trace=True)
        for layer, p, result, trace in zip(network.layers, params, output.results, output.traces):
            overflowed = trace.overflowed.cpu().numpy()
            if not overflowed.any():
                continue
            v_steps = trace.v_steps.cpu().numpy()
            event_ms = trace.event_ms.cpu().numpy()
            spikes = trace.spike_mask.cpu().numpy()
            vmin = result.v_unfitted_min.cpu().numpy()
            vmax = result.v_unfitted_max.cpu().numpy()
            w = int(p.i_V) + int(p.f_V)
            for neuron in np.nonzero(overflowed.any(axis=1))[0]:
                step = int(np.argmax(overflowed[neuron]))
                channel, y, x = _neuron_position(layer, int(neuron))
                events.append({
                    "sample": int(i), "layer": layer.name, "channel": channel, "y": y, "x": x,
                    "time_ms": float(event_ms[neuron, step]),
                    "v_before": int(v_steps[neuron, step - 1]) if step > 0 else 0,
                    "v_after": int(v_steps[neuron, step]),
                    "spiked": bool(spikes[neuron, step]),
                    "true_min": int(vmin[neuron]), "true_max": int(vmax[neuron]),
                    "register_range": [-2 ** (w - 1), 2 ** (w - 1) - 1]})
                if len(events) >= MAX_OVERFLOW_EVENTS:
                    return events
    return events


def overflow_summary(network, decoder, params, round_mode, raw, batch_size: int, policies: dict,
                     out, *, device=None) -> dict:
    """Overflowed samples per layer, headroom and, unless a layer saturates, the fewest
    extra register bits that remove every overflow and where the overflows happened
    (example/quant_run.py:213-240)."""
    names = [layer.name for layer in network.layers]
    summary = {"overflowed_samples": {n: int(out.overflowed[:, i].sum()) for i, n in enumerate(names)},
               "headroom_bits": dict(zip(names, headroom_bits(params, out)))}
    if any(OverflowMode(p.overflow_mode) is OverflowMode.SATURATE for p in params):
        return summary
    extra, rounds = min_extra_bits(network, decoder, params, round_mode, raw, batch_size,
                                   policies, out, device=device)
    return {**summary, "min_extra_bits": dict(zip(names, extra)), "min_extra_bits_rounds": rounds,
            "overflow_events": overflow_events(network, params, round_mode, raw, out)}
