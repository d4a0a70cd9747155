"""Model files: a network description plus its weights (float) or quantized parameters in
one .npz, in the on-disk format of the reference (salt_core/io.py:17-21, 121-180), so a
model folder written by either side loads in the other.

An archive is a flat name -> array map with two kinds of entries:

* JSON sections, each a 0-d unicode array holding one JSON object with a "format" field:
  "__network__" = {"format": 1, "input_shape": [...], "layers": [{"type": "conv" | "fc",
  <the layer's dataclass fields in declaration order>}, ...]}, and, in quantized files,
  "__quant__" = {"format": 1, "round_mode": ..., "layers": {name: {"f_a", "f_V", "i_V",
  "overflow_mode"}}, "metadata": {...}}.
* arrays: float files one per layer under the layer's name; quantized files
  "<layer>/q", "<layer>/decay_table_int", "<layer>/v_th_int" (absent for no threshold)
  and "<layer>/scale".

Reading uses numpy's loader with pickles refused, so a file executes nothing.  The error
texts of the reference are kept (callers match on them); a quantized model whose
thresholds are not positive is refused when it is loaded, naming the layer and channel,
since this path does not run such thresholds.
"""
from __future__ import annotations

import dataclasses
import json
import os
from collections.abc import Iterable, Mapping, Sequence
from typing import Any, NamedTuple

import numpy as np

from salt_amd.layers import ConvLayer, FCLayer
from salt_amd.network import Network
from salt_amd.quant.fixed_point import OverflowMode, RoundMode
from salt_amd.quant.params import QuantizedLayerParams

FORMAT_VERSION = 1
NETWORK_KEY = "__network__"
QUANT_KEY = "__quant__"

# description "type" of each layer class
_KIND_BY_CLASS = {ConvLayer: "conv", FCLayer: "fc"}
_CLASS_BY_KIND = {kind: cls for cls, kind in _KIND_BY_CLASS.items()}
# per-layer entries of a quantized archive: arrays "<layer>/<field>" (v_th_int optional)
# and the integer settings kept in the __quant__ section
_PARAM_ARRAYS = ("q", "decay_table_int", "v_th_int", "scale")
_PARAM_INTS = ("f_a", "f_V", "i_V")


def _numpy(x) -> np.ndarray:
    """A host numpy array of x (numpy, a Python scalar or a torch tensor on any device)."""
    detach = getattr(x, "detach", None)
    return detach().cpu().numpy() if detach else np.asarray(x)


# ------------------------------------------------------------------ JSON sections

def _pack_section(obj: Mapping[str, Any]) -> np.ndarray:
    return np.asarray(json.dumps(obj))


def _require_format(section: Mapping[str, Any], what: str) -> None:
    if section.get("format") != FORMAT_VERSION:
        raise ValueError(f"{what}的 format 要是 {FORMAT_VERSION},拿到 {section.get('format')!r}")


def _unpack_section(arrays: Mapping[str, np.ndarray], key: str, what: str) -> dict:
    if key not in arrays:
        raise ValueError(f"沒有{what}欄位 {key!r}")
    return json.loads(str(arrays[key]))


# ------------------------------------------------------------------ network description

def network_to_dict(network: Network) -> dict[str, Any]:
    """The description: input shape and, per layer, its type and every dataclass field
    (capacities included), ready for JSON.  A layer of another class raises ValueError."""
    entries = []
    for layer in network.layers:
        kind = _KIND_BY_CLASS.get(type(layer))
        if kind is None:
            raise ValueError(f"{layer.name} 的型別 {type(layer).__name__} 不能序列化")
        entries.append({"type": kind, **dataclasses.asdict(layer)})
    return {"format": FORMAT_VERSION, "input_shape": list(network.input_shape), "layers": entries}


def network_from_dict(description: Mapping[str, Any]) -> Network:
    """The Network a description holds; another format or an unknown layer type raises
    ValueError."""
    _require_format(description, "網路描述")
    layers = []
    for entry in description["layers"]:
        fields = {k: v for k, v in entry.items() if k != "type"}
        cls = _CLASS_BY_KIND.get(entry["type"])
        if cls is None:
            raise ValueError(f"不認得的層 type {entry['type']!r}(可用:{list(_CLASS_BY_KIND)})")
        layers.append(cls(**fields))
    return Network(input_shape=description["input_shape"], layers=layers)


def _names_for(network: Network, count: int, what: str) -> list[str]:
    """The layer names that key an archive's arrays: one entry per layer (count), names
    unique and never NETWORK_KEY; otherwise ValueError."""
    names = [layer.name for layer in network.layers]
    if count != len(names):
        raise ValueError(f"{what}有 {count} 份,網路有 {len(names)} 層")
    if NETWORK_KEY in names or len(set(names)) < len(names):
        raise ValueError(f"層名要不重複、而且不能是 {NETWORK_KEY!r},拿到 {names}")
    return names


def _described(network: Network, entries: Iterable[tuple[str, Any]]) -> dict[str, np.ndarray]:
    arrays = {key: _numpy(value) for key, value in entries}
    arrays[NETWORK_KEY] = _pack_section(network_to_dict(network))
    return arrays


def _network_of(arrays: Mapping[str, np.ndarray]) -> Network:
    return network_from_dict(_unpack_section(arrays, NETWORK_KEY, "網路描述"))


# ------------------------------------------------------------------ float weights

def weights_to_arrays(network: Network, weights: Sequence) -> dict[str, np.ndarray]:
    """Archive entries of a float model: each layer's weights under its name, plus the
    description (salt_core/io.py:87-97)."""
    names = _names_for(network, len(weights), "權重")
    return _described(network, zip(names, weights))


def weights_from_arrays(arrays: Mapping[str, np.ndarray]) -> tuple[Network, tuple[np.ndarray, ...]]:
    """(network, weights in layer order) of a float model's entries (an npz or a dict)."""
    network = _network_of(arrays)
    return network, tuple(np.asarray(arrays[layer.name]) for layer in network.layers)


def save_weights(path: str | os.PathLike, network: Network, weights: Sequence) -> None:
    np.savez(path, **weights_to_arrays(network, weights))


def load_weights(path: str | os.PathLike) -> tuple[Network, tuple[np.ndarray, ...]]:
    with np.load(path) as arrays:
        return weights_from_arrays(arrays)


# ------------------------------------------------------------------ quantized models

class QuantizedModel(NamedTuple):
    """What load_quantized returns (salt_core/io.py:121-126)."""
    network: Network
    params: tuple[QuantizedLayerParams, ...]  # in layer order
    round_mode: RoundMode
    metadata: dict[str, Any]


def save_quantized(path: str | os.PathLike, network: Network,
                   params: Sequence[QuantizedLayerParams], round_mode: RoundMode | str,
                   metadata: Mapping[str, Any]) -> None:
    """A quantized model as one archive that the integer path runs without float weights
    (the layout of salt_core/io.py:129-153).  metadata must be JSON-serialisable
    (TypeError otherwise); a layer count or naming problem raises ValueError."""
    names = _names_for(network, len(params), "量化參數")
    entries, settings = [], {}
    for name, p in zip(names, params):
        for field in _PARAM_ARRAYS:
            value = getattr(p, field)
            if value is not None:
                entries.append((f"{name}/{field}", value))
        settings[name] = {**{k: int(getattr(p, k)) for k in _PARAM_INTS},
                          "overflow_mode": OverflowMode(p.overflow_mode).value}
    arrays = _described(network, entries)
    arrays[QUANT_KEY] = _pack_section({"format": FORMAT_VERSION,
                                       "round_mode": RoundMode(round_mode).value,
                                       "layers": settings, "metadata": dict(metadata)})
    np.savez(path, **arrays)


def _refuse_nonpositive_thresholds(layer, v_th: np.ndarray | None) -> None:
    """A threshold <= 0 fires on every pad, catch-up and identity column of the reference's
    queue (salt_core/quant/scan.py:46-51), so its results depend on the capacities; this
    path refuses it, naming the first such channel (and neuron, for per-neuron ones)."""
    if v_th is None:
        return
    flat = np.asarray(v_th).reshape(-1)
    bad = np.flatnonzero(flat <= 0)
    if bad.size == 0:
        return
    i = int(bad[0])
    if flat.size == 1:
        where = "its scalar threshold"
    elif flat.size == layer.n_neurons and flat.size != getattr(layer, "oc", flat.size):
        plane = layer.n_neurons // layer.oc
        where = f"channel {i // plane} (neuron {i})"
    else:
        where = f"channel {i}"
    raise ValueError(f"{layer.name}: v_th_int = {int(flat[i])} <= 0 at {where}; thresholds must "
                     "be positive on this path (a non-positive one fires on the queue's pad, "
                     "catch-up and identity columns, so the reference's result would depend on "
                     "its capacities)")


def load_quantized(path: str | os.PathLike) -> QuantizedModel:
    """Reads a save_quantized archive.  A missing description or quant section, another
    format, or a threshold <= 0 raises ValueError."""
    with np.load(path) as arrays:
        network = _network_of(arrays)
        quant = _unpack_section(arrays, QUANT_KEY, "量化設定")
        _require_format(quant, "量化設定")
        params = []
        for layer in network.layers:
            stored = {f: np.asarray(arrays[f"{layer.name}/{f}"]) for f in _PARAM_ARRAYS
                      if f"{layer.name}/{f}" in arrays}
            _refuse_nonpositive_thresholds(layer, stored.get("v_th_int"))
            settings = quant["layers"][layer.name]
            params.append(QuantizedLayerParams(
                q=stored["q"], decay_table_int=stored["decay_table_int"],
                v_th_int=stored.get("v_th_int"), scale=stored["scale"],
                **{k: settings[k] for k in _PARAM_INTS},
                overflow_mode=OverflowMode(settings["overflow_mode"])))
    return QuantizedModel(network=network, params=tuple(params),
                          round_mode=RoundMode(quant["round_mode"]), metadata=quant["metadata"])
