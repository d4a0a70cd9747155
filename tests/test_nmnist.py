"""N-MNIST reader (salt_amd.data): 40-bit AER decoding against the hand-decoded sample of
data/tests/test_nmnist.py:22-29 and the format's field limits, the seeded train/val
partition, split padding and truncation, determinism, and InputEvents conversion.  Runs
on a synthetic dataset tree (the dataset itself is not shipped).  CPU only."""
import os

import numpy as np
import pytest

from helpers import encode_aer, write_nmnist_tree
from salt_amd.data import (IMG_SIZE, NMNISTDataset, decode_aer, decode_bin_file, list_files,
                           split_input_events, take_input_events)

# Train/0/00002.bin, first 10 events decoded by hand (data/tests/test_nmnist.py:24-29)
KNOWN_X = [10, 33, 12, 33, 14, 16, 7, 1, 16, 18]
KNOWN_Y = [30, 20, 27, 3, 23, 10, 30, 28, 11, 19]
KNOWN_C = [1, 1, 1, 1, 0, 0, 1, 1, 0, 1]
KNOWN_T_US = [937, 1030, 1052, 2078, 2383, 3189, 4003, 4975, 6609, 6678]


def test_decode_known_sample(tmp_path):
    path = tmp_path / "00002.bin"
    path.write_bytes(encode_aer(KNOWN_X, KNOWN_Y, KNOWN_C, KNOWN_T_US))
    x, y, c, t = decode_bin_file(str(path))
    assert x.tolist() == KNOWN_X and y.tolist() == KNOWN_Y and c.tolist() == KNOWN_C
    assert t.tolist() == [0, 1, 1, 2, 2, 3, 4, 4, 6, 6]
    assert all(a.dtype == np.int32 for a in (x, y, c, t))


def test_decode_field_limits():
    """Every timestamp bit is read (23 bits: 0x7FFFFF us -> 8388 ms), the polarity bit is
    not part of the time, and the time is floored."""
    raw = np.frombuffer(bytes([0, 0, 0xFF, 0xFF, 0xFF,      # c=1, t = 2^23 - 1 us
                               33, 33, 0x7F, 0xFF, 0xFF,    # c=0, t = 2^23 - 1 us
                               1, 2, 0x80, 0x03, 0xE7,      # c=1, t = 999 us -> 0 ms
                               1, 2, 0x00, 0x03, 0xE8]),    # c=0, t = 1000 us -> 1 ms
                        np.uint8)
    x, y, c, t = decode_aer(raw)
    assert c.tolist() == [1, 0, 1, 0]
    assert t.tolist() == [8388, 8388, 0, 1]
    assert x.tolist() == [0, 33, 1, 1] and y.tolist() == [0, 33, 2, 2]


def test_decode_rejects_bad_files(tmp_path):
    with pytest.raises(ValueError, match="5 的倍數"):
        decode_aer(np.zeros(7, np.uint8))
    with pytest.raises(ValueError, match="座標超出"):
        decode_aer(np.array([34, 0, 0, 0, 0], np.uint8))
    assert decode_aer(np.zeros(0, np.uint8))[0].shape == (0,)


@pytest.fixture(scope="module")
def tree(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("nmnist"))
    return root, write_nmnist_tree(root, per_digit_train=10, per_digit_test=3)


def test_list_files_order_and_labels(tree):
    root, _ = tree
    files, labels = list_files(root, "Test")
    assert len(files) == 30 and labels.tolist() == sorted(labels.tolist())
    assert [os.path.basename(os.path.dirname(f)) for f in files] == [str(l) for l in labels]
    for d in range(10):
        names = [f for f, l in zip(files, labels) if l == d]
        assert names == sorted(names)


def test_train_val_pools(tree):
    root, _ = tree
    ds = NMNISTDataset(root, max_events=100)
    train, train_labels, val, val_labels = ds._train_val_pools()
    assert len(train) + len(val) == 100 and len(val) == 10
    assert set(train).isdisjoint(val)
    assert len(train_labels) == len(train) and len(val_labels) == len(val)
    assert ds._train_val_pools() is ds._train_val_pools()
    assert (ds.pool_size("train"), ds.pool_size("val"), ds.pool_size("test")) == (90, 10, 30)
    assert NMNISTDataset(root, 100, val_fraction=0.25).pool_size("val") == 25
    # the partition depends on val_split_seed only
    other = NMNISTDataset(root, 100, val_split_seed=1)._train_val_pools()[2]
    assert other != val and sorted(NMNISTDataset(root, 50)._train_val_pools()[2]) == sorted(val)


def test_build_split_padding_truncation_and_contents(tree):
    root, files = tree
    m = 100
    ds = NMNISTDataset(root, max_events=m)
    split = ds.build_split(seed=3, n_samples=12, which="train")
    picked, labels = ds.sample_files(3, 12, "train")
    assert split.event_times.shape == (12, m) and split.labels_onehot.shape == (12, 10)
    assert np.array_equal(split.labels, labels)
    assert np.array_equal(split.labels_onehot.argmax(axis=1), split.labels)
    truncated = padded = 0
    for i, path in enumerate(picked):
        x, y, c, t_us = files[path]
        n = min(len(x), m)
        assert split.n_real_events[i] == n
        assert np.array_equal(split.x[i, :n], x[:n]) and np.array_equal(split.c[i, :n], c[:n])
        assert np.array_equal(split.event_times[i, :n], t_us[:n] // 1000)
        if n < m:
            padded += 1
            assert not split.x[i, n:].any() and not split.y[i, n:].any() and not split.c[i, n:].any()
            assert (split.event_times[i, n:] == t_us[n - 1] // 1000).all()
        else:
            truncated += len(x) > m
    assert truncated and padded


def test_build_split_determinism(tree):
    root, _ = tree
    ds = NMNISTDataset(root, max_events=80)
    a = ds.build_split(seed=5, n_samples=8, which="val")
    b = NMNISTDataset(root, max_events=80).build_split(seed=5, n_samples=8, which="val")
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    # n samples of a seed are the first n of a larger draw
    big = ds.build_split(seed=5, n_samples=10, which="val")
    assert np.array_equal(big.labels[:8], a.labels) and np.array_equal(big.x[:8], a.x)
    assert ds.sample_files(6, 8, "val")[0] != ds.sample_files(5, 8, "val")[0]
    with pytest.raises(ValueError, match="超過上限"):
        ds.build_split(seed=0, n_samples=11, which="val")
    with pytest.raises(ValueError, match="which"):
        ds.build_split(seed=0, n_samples=1, which="dev")


def test_constructor_arguments(tree):
    root, _ = tree
    with pytest.raises(TypeError):
        NMNISTDataset(root)  # max_events has no default
    with pytest.raises(ValueError):
        NMNISTDataset(root, max_events=0)
    with pytest.raises(ValueError):
        NMNISTDataset(root, max_events=10, val_fraction=1.0)
    assert NMNISTDataset(root, max_events=37).build_split(0, 2, "test").x.shape == (2, 37)


def test_split_input_events(tree):
    root, _ = tree
    split = NMNISTDataset(root, max_events=90).build_split(seed=1, n_samples=6, which="test")
    raw = split_input_events(split, (2, IMG_SIZE, IMG_SIZE))
    assert np.array_equal(raw.source_idx, split.c * 1156 + split.y * 34 + split.x)
    assert np.array_equal(raw.event_times, split.event_times)
    sub = take_input_events(raw, slice(2, 5))
    assert np.array_equal(sub.source_idx, raw.source_idx[2:5])
    assert np.array_equal(sub.n_real_events, raw.n_real_events[2:5])
