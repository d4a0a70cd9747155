"""A quantized conv layer as the $readmemh text files the SALT-FPGA conv RTL loads (the
files of salt_core/fpga_export.py): one value per line, each a fixed ceil(width/4) hex
digits, zero-padded.

* <layer>_weight.mem: line oc*C + c holds the K*K taps of that (output, input) channel
  pair as one word, tap ky*K + kx in bits [tap*b, (tap+1)*b) as b-bit two's complement.
* <layer>_threshold.mem: one threshold per output channel, (i_V + f_V)-bit two's
  complement.
* <layer>_decay.mem: line dt-1 holds the decay code A[dt], f_a-bit unsigned.

Every range and shape check of a layer runs before any of its files is written.  Error
texts are the reference's.
"""
from __future__ import annotations

import os
from collections.abc import Sequence
from pathlib import Path

import numpy as np


def hex_line(value: int, width: int) -> str:
    """A width-bit unsigned value as ceil(width/4) hex digits."""
    if width < 1:
        raise ValueError(f"位元寬要至少 1,拿到 {width}")
    if value < 0 or value >> width:
        raise ValueError(f"{value} 超出 {width} 位元無號範圍")
    return format(value, f"0{-(-width // 4)}x")


def twos_complement(value: int, width: int) -> int:
    """The width-bit two's-complement pattern of a signed value (range checked by the
    caller)."""
    return int(value) % (1 << width)


def _as_patterns(values, width: int, what: str) -> list[int]:
    """Signed values -> their width-bit two's-complement patterns (Python ints, any
    width); a value outside the signed range, or width < 1, raises ValueError."""
    if width < 1:
        raise ValueError(f"{what}的位元寬要至少 1,拿到 {width}")
    arr = np.asarray(values)
    lo, hi = -(1 << (width - 1)), (1 << (width - 1)) - 1
    if arr.size and not (lo <= arr.min() and arr.max() <= hi):
        raise ValueError(f"{what} 範圍 {arr.min()} ~ {arr.max()} 超出 {width} 位元二補數 "
                         f"{lo} ~ {hi}")
    return [twos_complement(v, width) for v in arr.reshape(-1).tolist()]


def conv_weight_lines(q, weight_width: int) -> list[str]:
    """The weight file's lines for codes q of shape (OC, C, K, K)."""
    q = np.asarray(q)
    if q.ndim != 4 or q.shape[2] != q.shape[3]:
        raise ValueError(f"q 要是 (OC, C, K, K),拿到形狀 {q.shape}")
    taps = q.shape[2] * q.shape[3]
    patterns = _as_patterns(q, weight_width, "權重碼")
    lines = []
    for start in range(0, len(patterns), taps):
        word = 0
        for p in reversed(patterns[start:start + taps]):  # the last tap is the top field
            word = (word << weight_width) | p
        lines.append(hex_line(word, taps * weight_width))
    return lines


def channel_thresholds(v_th_int, out_channels: int) -> np.ndarray:
    """One threshold per output channel from a scalar or a per-neuron array (neuron
    oc*H*W + y*W + x); a channel whose neurons disagree raises ValueError."""
    v = np.asarray(v_th_int)
    if v.ndim == 0:
        return np.full(out_channels, v.item())
    if v.ndim != 1 or v.size % out_channels:
        raise ValueError(f"v_th_int 形狀 {v.shape} 不能分成 {out_channels} 個 output channel")
    rows = v.reshape(out_channels, -1)
    uneven = np.flatnonzero(rows.min(axis=1) != rows.max(axis=1))
    if uneven.size:
        raise ValueError(f"output channel {uneven.tolist()} 的門檻不全相同")
    return rows[:, 0].copy()


def threshold_lines(thresholds, membrane_width: int) -> list[str]:
    """Per-channel thresholds as membrane_width-bit two's-complement lines."""
    return [hex_line(p, membrane_width)
            for p in _as_patterns(thresholds, membrane_width, "門檻")]


def decay_lines(decay_table_int, decay_frac_width: int) -> list[str]:
    """Decay codes as decay_frac_width-bit unsigned lines (line dt-1 = A[dt])."""
    return [hex_line(int(a), decay_frac_width) for a in np.asarray(decay_table_int).tolist()]


def write_mem(path: str | os.PathLike, lines: Sequence[str]) -> None:
    """Lines to a text file, each ended by a newline."""
    with open(path, "w", encoding="ascii", newline="\n") as f:
        f.writelines(line + "\n" for line in lines)


def write_conv_layer_mem(out_dir: str | os.PathLike, layer, params, weight_width: int
                         ) -> dict[str, Path]:
    """Writes <name>_weight.mem, <name>_threshold.mem and <name>_decay.mem of one conv
    layer into out_dir (created if needed); returns {"weight" | "threshold" | "decay":
    path}.  Shape and range problems raise ValueError before anything is written."""
    q = np.asarray(params.q)
    geometry = (layer.oc, layer.ic, layer.k, layer.k)
    if q.shape != geometry:
        raise ValueError(f"{layer.name} 的 q 形狀 {q.shape},層的幾何是 {geometry}")
    if params.v_th_int is None:
        raise ValueError(f"{layer.name} 沒有門檻,conv 層要能 fire")
    v_th = np.asarray(params.v_th_int)
    n_neurons = layer.oc * layer.h_out * layer.w_out
    if v_th.ndim != 0 and v_th.shape != (n_neurons,):
        raise ValueError(f"{layer.name} 的 v_th_int 形狀 {v_th.shape},神經元數 {n_neurons}")
    files = {"weight": conv_weight_lines(q, weight_width),
             "threshold": threshold_lines(channel_thresholds(v_th, layer.oc),
                                          params.i_V + params.f_V),
             "decay": decay_lines(params.decay_table_int, params.f_a)}
    target = Path(out_dir)
    target.mkdir(parents=True, exist_ok=True)
    written = {}
    for kind, lines in files.items():
        written[kind] = target / f"{layer.name}_{kind}.mem"
        write_mem(written[kind], lines)
    return written
