"""Model files: Network <-> description dict, and weights (float or quantized) stored with
the description in one .npz -- the on-disk format of salt_core/io.py, so that a model
folder written by the reference (model.npz) loads here and the other way round.

Format (salt_core/io.py:17-21, 121-180):
  "__network__"  0-d unicode array: JSON {"format": 1, "input_shape": [...], "layers":
                 [{"type": "conv" | "fc", <every dataclass field of the layer>}, ...]}
  quantized files add
  "__quant__"    0-d unicode array: JSON {"format": 1, "round_mode": ..., "layers":
                 {name: {"f_a", "f_V", "i_V", "overflow_mode"}}, "metadata": {...}}
  "<layer>/q", "<layer>/decay_table_int", "<layer>/v_th_int" (absent when None),
  "<layer>/scale"
  float-weight files hold one array per layer under the layer's name instead.
Arrays load as numpy arrays with their stored dtypes; nothing is unpickled.
"""
from __future__ import annotations

import dataclasses
import json
import os
from collections.abc import Mapping, Sequence
from typing import Any, NamedTuple

import numpy as np

from salt_amd.layers import ConvLayer, FCLayer
from salt_amd.network import Network
from salt_amd.quant.fixed_point import OverflowMode, RoundMode
from salt_amd.quant.params import QuantizedLayerParams

FORMAT_VERSION = 1
NETWORK_KEY = "__network__"
QUANT_KEY = "__quant__"
_LAYER_TYPES = {"conv": ConvLayer, "fc": FCLayer}


def _host(x) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor
        return x.detach().cpu().numpy()
    return np.asarray(x)


def _layer_type(layer) -> str:
    for name, cls in _LAYER_TYPES.items():
        if type(layer) is cls:
            return name
    raise ValueError(f"{layer.name} 的型別 {type(layer).__name__} 不能序列化")


def network_to_dict(network: Network) -> dict[str, Any]:
    """Input shape plus every field of every layer (capacities included), JSON-ready
    (salt_core/io.py:40-48).  Unknown layer classes raise ValueError."""
    return {"format": FORMAT_VERSION,
            "input_shape": list(network.input_shape),
            "layers": [{"type": _layer_type(layer), **dataclasses.asdict(layer)}
                       for layer in network.layers]}


def network_from_dict(description: Mapping[str, Any]) -> Network:
    """Inverse of network_to_dict (salt_core/io.py:51-63); a wrong format or an unknown
    layer type raises ValueError."""
    if description.get("format") != FORMAT_VERSION:
        raise ValueError(f"網路描述的 format 要是 {FORMAT_VERSION},"
                         f"拿到 {description.get('format')!r}")
    layers = []
    for entry in description["layers"]:
        fields = dict(entry)
        kind = fields.pop("type")
        if kind not in _LAYER_TYPES:
            raise ValueError(f"不認得的層 type {kind!r}(可用:{list(_LAYER_TYPES)})")
        layers.append(_LAYER_TYPES[kind](**fields))
    return Network(input_shape=description["input_shape"], layers=layers)


def _checked_layer_names(network: Network, n_given: int, what: str) -> list[str]:
    """Layer names; raises ValueError when the count differs, names repeat or a name is
    NETWORK_KEY (salt_core/io.py:66-73)."""
    names = [layer.name for layer in network.layers]
    if n_given != len(names):
        raise ValueError(f"{what}有 {n_given} 份,網路有 {len(names)} 層")
    if len(set(names)) != len(names) or NETWORK_KEY in names:
        raise ValueError(f"層名要不重複、而且不能是 {NETWORK_KEY!r},拿到 {names}")
    return names


def _network_json(network: Network) -> np.ndarray:
    return np.asarray(json.dumps(network_to_dict(network)))


def _read_network(arrays: Mapping[str, np.ndarray]) -> Network:
    if NETWORK_KEY not in arrays:
        raise ValueError(f"沒有網路描述欄位 {NETWORK_KEY!r}")
    return network_from_dict(json.loads(str(arrays[NETWORK_KEY])))


def weights_to_arrays(network: Network, weights: Sequence) -> dict[str, np.ndarray]:
    """One array per layer under its name, plus the description (salt_core/io.py:87-97)."""
    names = _checked_layer_names(network, len(weights), "權重")
    arrays = {name: _host(w) for name, w in zip(names, weights)}
    arrays[NETWORK_KEY] = _network_json(network)
    return arrays


def weights_from_arrays(arrays: Mapping[str, np.ndarray]) -> tuple[Network, tuple[np.ndarray, ...]]:
    """Inverse of weights_to_arrays (salt_core/io.py:100-106)."""
    network = _read_network(arrays)
    return network, tuple(np.asarray(arrays[layer.name]) for layer in network.layers)


def save_weights(path: str | os.PathLike, network: Network, weights: Sequence) -> None:
    """salt_core/io.py:109-112."""
    np.savez(path, **weights_to_arrays(network, weights))


def load_weights(path: str | os.PathLike) -> tuple[Network, tuple[np.ndarray, ...]]:
    """salt_core/io.py:115-118."""
    with np.load(path) as arrays:
        return weights_from_arrays(arrays)


class QuantizedModel(NamedTuple):
    """load_quantized's result (salt_core/io.py:121-126)."""
    network: Network
    params: tuple[QuantizedLayerParams, ...]
    round_mode: RoundMode
    metadata: dict[str, Any]


def save_quantized(path: str | os.PathLike, network: Network,
                   params: Sequence[QuantizedLayerParams], round_mode: RoundMode | str,
                   metadata: Mapping[str, Any]) -> None:
    """A quantized model as one .npz that QuantBackend runs without float weights
    (salt_core/io.py:129-153).  metadata must be JSON-serialisable (json.dumps raises
    TypeError otherwise); layer-count or name problems raise ValueError."""
    names = _checked_layer_names(network, len(params), "量化參數")
    arrays = {NETWORK_KEY: _network_json(network)}
    layers_info = {}
    for name, p in zip(names, params):
        arrays[f"{name}/q"] = _host(p.q)
        arrays[f"{name}/decay_table_int"] = _host(p.decay_table_int)
        if p.v_th_int is not None:
            arrays[f"{name}/v_th_int"] = _host(p.v_th_int)
        arrays[f"{name}/scale"] = _host(p.scale)
        layers_info[name] = {"f_a": int(p.f_a), "f_V": int(p.f_V), "i_V": int(p.i_V),
                             "overflow_mode": OverflowMode(p.overflow_mode).value}
    arrays[QUANT_KEY] = np.asarray(json.dumps({
        "format": FORMAT_VERSION, "round_mode": RoundMode(round_mode).value,
        "layers": layers_info, "metadata": dict(metadata)}))
    np.savez(path, **arrays)


def load_quantized(path: str | os.PathLike) -> QuantizedModel:
    """Reads a save_quantized file (salt_core/io.py:156-180); a missing description or
    quant section, or a wrong format, raises ValueError."""
    with np.load(path) as arrays:
        network = _read_network(arrays)
        if QUANT_KEY not in arrays:
            raise ValueError(f"沒有量化設定欄位 {QUANT_KEY!r}")
        quant = json.loads(str(arrays[QUANT_KEY]))
        if quant.get("format") != FORMAT_VERSION:
            raise ValueError(f"量化設定的 format 要是 {FORMAT_VERSION},拿到 {quant.get('format')!r}")
        params = []
        for layer in network.layers:
            name, info = layer.name, quant["layers"][layer.name]
            v_th_key = f"{name}/v_th_int"
            params.append(QuantizedLayerParams(
                q=np.asarray(arrays[f"{name}/q"]),
                decay_table_int=np.asarray(arrays[f"{name}/decay_table_int"]),
                v_th_int=np.asarray(arrays[v_th_key]) if v_th_key in arrays else None,
                scale=np.asarray(arrays[f"{name}/scale"]),
                f_a=info["f_a"], f_V=info["f_V"], i_V=info["i_V"],
                overflow_mode=OverflowMode(info["overflow_mode"])))
    return QuantizedModel(network=network, params=tuple(params),
                          round_mode=RoundMode(quant["round_mode"]), metadata=quant["metadata"])
