"""N-MNIST reader with the behaviour of data/src/nmnist.py: .bin decoding, the seeded
train/val partition of Train/, and padded, truncated sample splits.  Host-side numpy;
the arrays feed InputEvents (see salt_amd.data.events).

File format (the dataset's published 40-bit AER layout): 5 bytes per event, in time
order -- byte 0 = x, byte 1 = y, bit 7 of byte 2 = polarity, the low 7 bits of byte 2
followed by bytes 3 and 4 = a 23-bit timestamp in microseconds.  Times become integer
milliseconds by floor division (t_us // 1000).
"""
from __future__ import annotations

import glob
import os
from typing import NamedTuple

import numpy as np

IMG_SIZE = 34                                        # data/src/nmnist.py:16
CHANNEL_NAMES: tuple[str, ...] = ("off", "on")       # channel c = polarity (:19)
CLASS_NAMES: tuple[str, ...] = tuple(str(d) for d in range(10))
_DEFAULT_VAL_FRACTION = 0.1                          # :25-26
_DEFAULT_VAL_SPLIT_SEED = 0


def decode_aer(raw: np.ndarray, where: str = "AER data") -> tuple[np.ndarray, ...]:
    """Bytes of one file -> (x, y, c, t_ms) int32 in file order
    (data/src/nmnist.py:29-49).  Raises ValueError when the length is not a multiple of 5
    or a coordinate lies outside [0, 34)."""
    raw = np.asarray(raw, dtype=np.uint8).reshape(-1)
    if raw.size % 5 != 0:
        raise ValueError(f"{where} 檔案大小 {raw.size} bytes 不是 5 的倍數,"
                         f"不符合 N-MNIST 40-bit AER 格式")
    ev = raw.reshape(-1, 5)
    x = ev[:, 0].astype(np.int32)
    y = ev[:, 1].astype(np.int32)
    if ev.shape[0] and (x.max() >= IMG_SIZE or y.max() >= IMG_SIZE):
        raise ValueError(f"{where} 座標超出 [0,{IMG_SIZE}) 範圍:"
                         f"x=[{x.min()},{x.max()}], y=[{y.min()},{y.max()}]")
    c = (ev[:, 2] >> 7).astype(np.int32)
    t_us = ((ev[:, 2].astype(np.uint32) & 0x7F) << 16) | (ev[:, 3].astype(np.uint32) << 8) \
        | ev[:, 4].astype(np.uint32)
    return x, y, c, (t_us // 1000).astype(np.int32)


def decode_bin_file(path: str) -> tuple[np.ndarray, ...]:
    """One .bin file -> (x, y, c, t_ms), see decode_aer."""
    return decode_aer(np.fromfile(path, dtype=np.uint8), path)


def list_files(dataset_root: str, split_dir: str) -> tuple[list[str], np.ndarray]:
    """Every .bin under split_dir/<digit>/ with its label, ordered by (digit, file name)
    (data/src/nmnist.py:52-61)."""
    files: list[str] = []
    labels: list[int] = []
    for digit in range(len(CLASS_NAMES)):
        found = sorted(glob.glob(os.path.join(dataset_root, split_dir, str(digit), "*.bin")))
        files.extend(found)
        labels.extend([digit] * len(found))
    return files, np.asarray(labels, dtype=np.int32)


class NMNISTSplit(NamedTuple):
    """data/src/nmnist.py:64-71 (numpy arrays)."""
    event_times: np.ndarray    # (N, max_events) int32 ms, non-decreasing
    x: np.ndarray              # (N, max_events) int32
    y: np.ndarray              # (N, max_events) int32
    c: np.ndarray              # (N, max_events) int32, 0 = OFF, 1 = ON
    n_real_events: np.ndarray  # (N,) int32
    labels: np.ndarray         # (N,) int32
    labels_onehot: np.ndarray  # (N, 10) float32


class NMNISTDataset:
    """One preprocessing setup (truncation length, train/val partition) from which
    splits are drawn (data/src/nmnist.py:74-177).

    dataset_root: directory holding Train/ and Test/, each with 0..9 subdirectories.
    max_events: events per sample; later events are cut, short samples padded.
    val_fraction / val_split_seed: the partition of Train/ into train and val pools.
    """

    def __init__(self, dataset_root: str, max_events: int,
                 val_fraction: float = _DEFAULT_VAL_FRACTION,
                 val_split_seed: int = _DEFAULT_VAL_SPLIT_SEED) -> None:
        if max_events <= 0:
            raise ValueError(f"max_events 必須是正整數,拿到 {max_events}")
        if not 0.0 < val_fraction < 1.0:
            raise ValueError(f"val_fraction 必須落在 (0, 1),拿到 {val_fraction}")
        self.dataset_root = str(dataset_root)
        self.max_events = int(max_events)
        self.val_fraction = float(val_fraction)
        self.val_split_seed = int(val_split_seed)
        self._pools = None

    def _train_val_pools(self):
        """(train_files, train_labels, val_files, val_labels): Train/ permuted by
        RandomState(val_split_seed), the first round(n * val_fraction) files are val.
        Computed once per instance."""
        if self._pools is None:
            files, labels = list_files(self.dataset_root, "Train")
            perm = np.random.RandomState(self.val_split_seed).permutation(len(files))
            n_val = int(round(len(files) * self.val_fraction))
            val_idx, train_idx = perm[:n_val], perm[n_val:]
            self._pools = ([files[i] for i in train_idx], labels[train_idx],
                           [files[i] for i in val_idx], labels[val_idx])
        return self._pools

    def _pool(self, which: str) -> tuple[list[str], np.ndarray]:
        if which == "train":
            files, labels, _, _ = self._train_val_pools()
        elif which == "val":
            _, _, files, labels = self._train_val_pools()
        elif which == "test":
            files, labels = list_files(self.dataset_root, "Test")
        else:
            raise ValueError(f"which 必須是 'train'/'val'/'test',拿到 {which!r}")
        return files, labels

    def pool_size(self, which: str) -> int:
        return len(self._pool(which)[0])

    def sample_files(self, seed: int, n_samples: int, which: str) -> tuple[list[str], np.ndarray]:
        """The files and labels build_split draws: RandomState(seed).choice(pool, n,
        replace=False), so n samples of a seed are the first n of a larger draw."""
        files, labels = self._pool(which)
        if n_samples > len(files):
            raise ValueError(f"which={which!r} 的 pool 只有 {len(files)} 筆,"
                             f"要求 n_samples={n_samples} 超過上限")
        idx = np.random.RandomState(seed).choice(len(files), size=n_samples, replace=False)
        return [files[i] for i in idx], labels[idx].astype(np.int32)

    def build_split(self, seed: int, n_samples: int, which: str) -> NMNISTSplit:
        """n_samples files of the `which` pool (data/src/nmnist.py:130-177), each cut to
        its first max_events events or padded: coordinates 0, times = the last real
        event's time (0 for an empty file)."""
        files, labels = self.sample_files(seed, n_samples, which)
        m = self.max_events
        times = np.zeros((n_samples, m), np.int32)
        xs = np.zeros((n_samples, m), np.int32)
        ys = np.zeros((n_samples, m), np.int32)
        cs = np.zeros((n_samples, m), np.int32)
        n_real = np.zeros(n_samples, np.int32)
        for i, path in enumerate(files):
            x, y, c, t = decode_bin_file(path)
            n = min(x.shape[0], m)
            times[i, :n], xs[i, :n], ys[i, :n], cs[i, :n] = t[:n], x[:n], y[:n], c[:n]
            times[i, n:] = t[n - 1] if n > 0 else 0
            n_real[i] = n
        onehot = np.eye(len(CLASS_NAMES), dtype=np.float32)[labels]
        return NMNISTSplit(event_times=times, x=xs, y=ys, c=cs, n_real_events=n_real,
                           labels=labels, labels_onehot=onehot)
