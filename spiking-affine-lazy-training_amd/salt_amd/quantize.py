"""Quantized model folders: re-running and checking them (example/quantize.py:306-366).

A folder holds model.npz (salt_amd.io.save_quantized format, metadata recording how the
verify samples were drawn from N-MNIST), reference.npz (the per-sample reference fields
plus labels) and report.yaml.

  python -m salt_amd.quantize --check QUANT_DIR --dataset-root N-MNIST/
      re-runs the verify samples on the GPU and compares every per-sample field with
      reference.npz; exit status 0 when all are equal, 1 otherwise.
  python -m salt_amd.quantize --eval QUANT_DIR --dataset-root N-MNIST/ [--which test|val]
      [--n N] [--seed S]
      runs `which` samples, growing capacities until every sample fits, and writes
      eval/<which>.yaml and eval/<which>_outputs.npz into the folder.
"""
from __future__ import annotations

import argparse
import datetime
import os
import sys

import numpy as np

from salt_amd.capacity import GrowthPolicy
from salt_amd.data.events import split_input_events
from salt_amd.data.nmnist import NMNISTDataset
from salt_amd.decoder import build_decoder
from salt_amd.io import load_quantized
from salt_amd.quant_run import (overflow_summary, quant_forward_split, reference_arrays,
                                run_until_fits)

MODEL_FILENAME = "model.npz"
REFERENCE_FILENAME = "reference.npz"
REPORT_FILENAME = "report.yaml"
EVAL_DIRNAME = "eval"


def build_split(dataset_root: str, max_events: int, which: str, seed: int, n: int):
    """n samples of the `which` pool (example/quantize.py:139-142)."""
    return NMNISTDataset(dataset_root, max_events=max_events).build_split(
        seed=seed, n_samples=n, which=which)


def split_of(dataset_root: str, data_meta: dict, part: str):
    """The verify or calibration sampling recorded in a model's metadata
    (example/quantize.py:162-165)."""
    s = data_meta[part]
    return build_split(dataset_root, data_meta["max_events"], s["split"], s["seed"], s["n"])


def check(quant_dir: str, dataset_root: str, *, device=None) -> int:
    """Re-runs quant_dir's model on its verify samples and compares every reference
    field per sample with reference.npz (example/quantize.py:306-330).  Returns 0 when
    everything is equal, 1 otherwise."""
    model = load_quantized(os.path.join(quant_dir, MODEL_FILENAME))
    with np.load(os.path.join(quant_dir, REFERENCE_FILENAME)) as npz:
        reference = dict(npz)
    split = split_of(dataset_root, model.metadata["data"], "verify")
    raw = split_input_events(split, model.network.input_shape)
    labels = np.asarray(split.labels)
    decoder = build_decoder({"decoder": model.metadata["decoder"]}, model.network.layers)
    out = quant_forward_split(model.network, decoder, model.params, model.round_mode, raw,
                              int(model.metadata["batch_size"]), device=device)
    n_diff = 0
    if not np.array_equal(labels, reference["labels"]):
        print("labels differ: the dataset or the sampling is not the one the folder was made with")
        n_diff += 1
    print(f"accuracy {float(np.mean(out.preds == labels)):.4f} "
          f"(reference {float(np.mean(reference['preds'] == reference['labels'])):.4f}, "
          f"n={labels.shape[0]})")
    for key, value in reference_arrays(out).items():
        diff = value != reference[key]
        idx = np.nonzero(diff.reshape(diff.shape[0], -1).any(axis=1))[0]
        print(f"{key} differs: {idx.size} samples {idx[:20].tolist()}")
        n_diff += idx.size
    return int(bool(n_diff))


def _capacity(network) -> dict:
    return {layer.name: dict(layer.capacity) for layer in network.layers
            if layer.capacity is not None}


def evaluate(quant_dir: str, dataset_root: str, which: str, n_samples: int | None, seed: int,
             *, device=None) -> dict:
    """`which` samples through the folder's model, capacities grown until every sample
    fits (the saved model is unchanged); writes eval/<which>.yaml and
    eval/<which>_outputs.npz (example/quantize.py:333-366)."""
    import yaml
    model = load_quantized(os.path.join(quant_dir, MODEL_FILENAME))
    meta = model.metadata
    if n_samples is None:
        n_samples = (NMNISTDataset(dataset_root, max_events=meta["data"]["max_events"])
                     .pool_size("test") if which == "test" else meta["data"]["val_size"])
    split = build_split(dataset_root, meta["data"]["max_events"], which, seed, n_samples)
    raw = split_input_events(split, model.network.input_shape)
    labels = np.asarray(split.labels)
    decoder = build_decoder({"decoder": meta["decoder"]}, model.network.layers)
    policies = {name: GrowthPolicy(**p) for name, p in meta["growth"].items()}
    batch_size = int(meta["batch_size"])
    network, out, n_regrow = run_until_fits(model.network, decoder, model.params,
                                            model.round_mode, raw, batch_size, policies,
                                            device=device)
    result = {
        "which": which, "n_samples": int(n_samples), "seed": int(seed),
        "accuracy": float(np.mean(out.preds == labels)),
        **overflow_summary(network, decoder, model.params, model.round_mode, raw, batch_size,
                           policies, out, device=device),
        "n_regrow": n_regrow,
        "capacity": _capacity(network),
        "timestamp": datetime.datetime.now().isoformat(timespec="seconds"),
    }
    eval_dir = os.path.join(quant_dir, EVAL_DIRNAME)
    os.makedirs(eval_dir, exist_ok=True)
    np.savez(os.path.join(eval_dir, f"{which}_outputs.npz"), labels=labels, **reference_arrays(out))
    with open(os.path.join(eval_dir, f"{which}.yaml"), "w", encoding="utf-8") as f:
        yaml.safe_dump(result, f, allow_unicode=True, sort_keys=False)
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--check", metavar="QUANT_DIR", help="re-run this folder and compare")
    ap.add_argument("--eval", metavar="QUANT_DIR", help="evaluate this folder on test or val")
    ap.add_argument("--dataset-root", required=True,
                    help="N-MNIST directory holding Train/ and Test/")
    ap.add_argument("--which", choices=("test", "val"), default="test")
    ap.add_argument("--n", type=int, default=None, help="--eval: number of samples")
    ap.add_argument("--seed", type=int, default=0, help="--eval: sampling seed")
    args = ap.parse_args(argv)
    if (args.check is None) == (args.eval is None):
        ap.error("give exactly one of --check and --eval")
    if args.check is not None:
        return check(args.check, args.dataset_root)
    import yaml
    print(yaml.safe_dump(evaluate(args.eval, args.dataset_root, args.which, args.n, args.seed),
                         allow_unicode=True, sort_keys=False))
    print(f"wrote {os.path.join(args.eval, EVAL_DIRNAME)}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
