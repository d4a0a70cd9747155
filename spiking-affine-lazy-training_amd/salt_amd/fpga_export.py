"""A quantized conv layer as the $readmemh hex text files of the SALT-FPGA conv RTL
(salt_core/fpga_export.py): packed weight words, per-output-channel thresholds, decay
table.  One value per line, fixed ceil(width/4) hex digits, zero-padded."""
from __future__ import annotations

import os
from collections.abc import Sequence
from pathlib import Path

import numpy as np


def hex_line(value: int, width: int) -> str:
    """A width-bit unsigned value as ceil(width/4) hex digits (fpga_export.py:15-24)."""
    if width < 1:
        raise ValueError(f"位元寬要至少 1,拿到 {width}")
    if not 0 <= value < (1 << width):
        raise ValueError(f"{value} 超出 {width} 位元無號範圍")
    return f"{value:0{(width + 3) // 4}x}"


def _checked_signed(values, width: int, what: str) -> np.ndarray:
    if width < 1:
        raise ValueError(f"{what}的位元寬要至少 1,拿到 {width}")
    values = np.asarray(values)
    low, high = -(1 << (width - 1)), (1 << (width - 1)) - 1
    if values.size and (values.min() < low or values.max() > high):
        raise ValueError(f"{what} 範圍 {values.min()} ~ {values.max()} 超出 {width} 位元二補數 "
                         f"{low} ~ {high}")
    return values.astype(object)


def twos_complement(value: int, width: int) -> int:
    """A signed value as its width-bit two's-complement bit pattern."""
    return int(value) & ((1 << width) - 1)


def conv_weight_lines(q, weight_width: int) -> list[str]:
    """Weight file lines (fpga_export.py:44-64): address oc*C + c holds one K*K*b-bit
    word, tap ky*K + kx at bit (ky*K + kx)*b.  q must be (OC, C, K, K) within b-bit two's
    complement."""
    q = np.asarray(q)
    if q.ndim != 4 or q.shape[2] != q.shape[3]:
        raise ValueError(f"q 要是 (OC, C, K, K),拿到形狀 {q.shape}")
    oc, ic, k, _ = q.shape
    codes = _checked_signed(q, weight_width, "權重碼").reshape(oc * ic, k * k)
    lines = []
    for kernel in codes:
        word = 0
        for tap, code in enumerate(kernel):
            word |= twos_complement(code, weight_width) << (tap * weight_width)
        lines.append(hex_line(word, k * k * weight_width))
    return lines


def channel_thresholds(v_th_int, out_channels: int) -> np.ndarray:
    """Per-neuron (or scalar) thresholds -> one per output channel; a channel whose
    neurons disagree raises ValueError (fpga_export.py:67-83)."""
    v_th_int = np.asarray(v_th_int)
    if v_th_int.ndim == 0:
        return np.full(out_channels, v_th_int.item())
    if v_th_int.ndim != 1 or v_th_int.size % out_channels != 0:
        raise ValueError(f"v_th_int 形狀 {v_th_int.shape} 不能分成 {out_channels} 個 output channel")
    per_channel = v_th_int.reshape(out_channels, -1)
    mismatched = np.flatnonzero((per_channel != per_channel[:, :1]).any(axis=1))
    if mismatched.size:
        raise ValueError(f"output channel {mismatched.tolist()} 的門檻不全相同")
    return per_channel[:, 0]


def threshold_lines(thresholds, membrane_width: int) -> list[str]:
    """Thresholds as membrane_width-bit two's complement (fpga_export.py:86-92)."""
    values = _checked_signed(thresholds, membrane_width, "門檻")
    return [hex_line(twos_complement(v, membrane_width), membrane_width) for v in values]


def decay_lines(decay_table_int, decay_frac_width: int) -> list[str]:
    """Decay codes, line dt-1 = A[dt], decay_frac_width-bit unsigned (fpga_export.py:95-100)."""
    return [hex_line(int(v), decay_frac_width) for v in np.asarray(decay_table_int)]


def write_mem(path: str | os.PathLike, lines: Sequence[str]) -> None:
    Path(path).write_text("".join(f"{line}\n" for line in lines), encoding="ascii")


def write_conv_layer_mem(out_dir: str | os.PathLike, layer, params, weight_width: int
                         ) -> dict[str, Path]:
    """<name>_weight.mem, <name>_threshold.mem (i_V + f_V bits) and <name>_decay.mem (f_a
    bits) of one conv layer (fpga_export.py:108-138).  Every check runs before any file
    is written."""
    q = np.asarray(params.q)
    if q.shape != (layer.oc, layer.ic, layer.k, layer.k):
        raise ValueError(f"{layer.name} 的 q 形狀 {q.shape},層的幾何是 "
                         f"{(layer.oc, layer.ic, layer.k, layer.k)}")
    if params.v_th_int is None:
        raise ValueError(f"{layer.name} 沒有門檻,conv 層要能 fire")
    v_th_int = np.asarray(params.v_th_int)
    n_neurons = layer.oc * layer.h_out * layer.w_out
    if v_th_int.ndim != 0 and v_th_int.shape != (n_neurons,):
        raise ValueError(f"{layer.name} 的 v_th_int 形狀 {v_th_int.shape},神經元數 {n_neurons}")
    contents = {
        "weight": conv_weight_lines(q, weight_width),
        "threshold": threshold_lines(channel_thresholds(v_th_int, layer.oc),
                                     params.i_V + params.f_V),
        "decay": decay_lines(np.asarray(params.decay_table_int), params.f_a),
    }
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    paths = {}
    for kind, lines in contents.items():
        paths[kind] = out_dir / f"{layer.name}_{kind}.mem"
        write_mem(paths[kind], lines)
    return paths
