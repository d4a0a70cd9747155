"""Output decoder of the integer path: membrane regression (salt_core/decoder.py:34-50).

The last layer does not fire (v_th_int = None, or a threshold it never reaches) and its
final registers, after QuantBackend.readout, are the class scores.  The reference's rate
and population decoders read the float path's soft spike values (s_value), which the
integer path has no counterpart for; quantized models always use membrane regression
(example/quantize.py:255-257).
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class MembraneRegressionDecoder:
    """scores = the last layer's v_final (salt_core/decoder.py:34-50)."""
    min_out_v_th: float = 1e6

    def decode(self, result):
        """(scores, metrics) of one sample or a batch: (v_final, {})."""
        return result.v_final, {}

    def validate(self, last_layer) -> None:
        if last_layer.v_th < self.min_out_v_th:
            raise ValueError(
                f"膜電位回歸要求輸出層近乎不 fire(v_th >= {self.min_out_v_th:g}),"
                f"但最後一層 {getattr(last_layer, 'name', '?')} 的 v_th={last_layer.v_th:g}")


def build_decoder(model_cfg: dict, layers=None) -> MembraneRegressionDecoder:
    """Decoder named by a model config's "decoder" key (example/models/conv_net.py:108-124);
    only membrane_regression (the default) exists on the integer path."""
    kind = model_cfg.get("decoder", "membrane_regression")
    if kind == "membrane_regression":
        return MembraneRegressionDecoder()
    if kind in ("rate", "population"):
        raise ValueError(f"decoder {kind!r} reads the float path's s_value; the integer "
                         "path supports membrane_regression only")
    raise ValueError(f"未知的 decoder 種類:{kind!r}(可用:membrane_regression / rate / population)")
