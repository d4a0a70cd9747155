#!/usr/bin/env python3
"""Benchmark: integer event-by-event forward (salt_core/quant semantics) on one MI355X.

Default workload: the N-MNIST-shaped network of the benchmark configuration 3 (conv
2->16 5x5 s2 -> conv 16->32 3x3 s2 -> FC 1568->10, 1024 synthetic streams of ~4500
events).  A step = one forward of the whole network over the batch, inputs resident in
HBM, every layer's spike stream, final registers and per-stream statistics written.

Prints one JSON line (the driver's contract).  value = layer-1 input events / second.
The step's output is checked bit for bit against the CPU oracle, whose timing on the
host cores is the cpu_baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "spiking-affine-lazy-training_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "input events/sec (batch, 1 MI355X) bit-exact vs salt_core/quant; % HBM/LDS roofline"
HBM_PEAK_GBS = 8000.0                     # MI355X HBM3E
LDS_PEAK_GBS = 256 * 128 * 2.4            # 256 CUs x 128 B/clk x 2.4 GHz = 78.6 TB/s
# Measured HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE, scaled by a copy
# of known size), one file per workload; each file names the commands that produced it.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_{workload}.json")
COPY_BYTES = 1 << 30                      # --copy-calibration: bytes read (and written)


def copy_calibration() -> int:
    """A plain device-to-device copy of COPY_BYTES, three times: the reference launch
    whose FETCH_SIZE / WRITE_SIZE readings scale the counters of the layer kernels."""
    import torch
    torch.cuda.set_device(0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 3}), flush=True)
    return 0


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of one layer kernel of one workload from the committed
    profile, or None when that workload has no traffic profile."""
    try:
        with open(TRAFFIC_FILE.format(workload=workload), encoding="utf-8") as f:
            return json.load(f)["per_launch_bytes"].get(kernel)
    except (OSError, KeyError, ValueError):
        return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def end_to_end(runner, w, dev, reps=5):
    """Host -> device -> host: the events copied from pinned host memory, the whole network
    in one salt_network_forward call, every layer's stream, registers and stats copied
    back; the PCIe-inclusive time of one batch (median of reps)."""
    import numpy as np
    import torch
    from salt_amd.stream import EventStream, unit_gain
    t_h = torch.from_numpy(np.ascontiguousarray(w.events.event_times, dtype=np.float32)).pin_memory()
    s_h = torch.from_numpy(np.ascontiguousarray(w.events.source_idx, dtype=np.int32)).pin_memory()
    n_h = torch.from_numpy(np.ascontiguousarray(w.events.n_real_events, dtype=np.int32)).pin_memory()
    outs_h = None
    times = []
    for _ in range(reps + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        t_d = t_h.to(dev, non_blocking=True)
        stream = EventStream(event_times=t_d, event_source_idx=s_h.to(dev, non_blocking=True),
                             event_gain=unit_gain(t_d), n_real_events=n_h.to(dev, non_blocking=True))
        outs = runner.run(stream)
        if outs_h is None:
            outs_h = [[torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
                       for x in (o.times, o.src, o.n, o.v_final, o.stats)] for o in outs]
        for o, hs in zip(outs, outs_h):
            for x, h in zip((o.times, o.src, o.n, o.v_final, o.stats), hs):
                h.copy_(x, non_blocking=True)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return float(np.median(times[1:])) * 1000.0


def conv_update_counts(layer, src, n_real):
    """Per stream, the number of (neuron, event) register updates of a conv layer: the
    valid candidate positions of every real event x output channels (numpy, host)."""
    import numpy as np
    K, S, P = layer.k, layer.s, layer.p
    hw = layer.h_in * layer.w_in
    L = src.shape[1]
    real = np.arange(L)[None, :] < n_real[:, None]
    rem = src % hw
    y, x = rem // layer.w_in, rem % layer.w_in

    def axis(i, o_max):
        lo = np.maximum(-((-(i + P - K + 1)) // S), 0)
        hi = np.minimum((i + P) // S, o_max - 1)
        return np.maximum(hi - lo + 1, 0)

    per_event = axis(y, layer.h_out) * axis(x, layer.w_out) * layer.oc
    return (per_event * real).sum(axis=1)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, help="benchmark configuration 1..5")
    ap.add_argument("--cpu-threads", type=int, default=0, help="oracle threads (0: all, max 16)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and the check")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the reference copy used to scale HBM traffic counters")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(streams would shard across GPUs with no communication; see DESIGN.md)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from salt_amd import workloads as W
    from salt_amd.runner import NetworkRunner

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    w = W.CONFIGS[args.config]()
    net = w.network
    runner = NetworkRunner(net, w.params, w.round_mode, dev)
    stream = net.input_stream(w.events, device=dev)
    n_events = int(w.events.n_real_events.sum())
    B, L = w.events.event_times.shape
    n_layers = len(net.layers)

    for _ in range(max(args.warmup, 1)):
        outs = runner.run(stream)
    torch.cuda.synchronize()
    fits = runner.check_fits(outs)

    # Timed region: K steps bracketed by synchronize, each one salt_layer_forward per
    # layer (the calls salt_network_forward makes), with HIP events around each layer's
    # launch on the stream the kernels run on (torch's current stream).
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_layers)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        outs = runner.run_layers(stream, around=lambda i, ph, k=k: ev[k][i][ph].record())
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = np.array([[ev[k][i][0].elapsed_time(ev[k][i][1]) for i in range(n_layers)]
                          for k in range(args.steps)]).mean(axis=0)
    ms_per_step = wall * 1000.0 / args.steps
    value = n_events / (ms_per_step / 1000.0)

    e2e_ms = end_to_end(runner, w, dev)

    # Algorithmic traffic of each layer (per launch): LDS = updates x (4 + 4 + weight bytes),
    # HBM = 8 B per input event + 8 B per spike + 4 B per final register + weights.
    host = [(o.src.cpu().numpy(), o.n.cpu().numpy()) for o in outs]
    in_src, in_n = w.events.source_idx, w.events.n_real_events
    per_layer = []
    for i, (layer, p, dp) in enumerate(zip(net.layers, w.params, runner.dev_params)):
        wbytes = dp.q_bits // 8
        n_in_events = int(np.minimum(in_n, in_src.shape[1]).sum())
        if hasattr(layer, "oc"):
            updates = int(conv_update_counts(layer, in_src, np.minimum(in_n, in_src.shape[1])).sum())
        else:
            updates = n_in_events * layer.n_out
        spikes = int(host[i][1].sum())
        lds = updates * (8 + wbytes)
        hbm = 8 * n_in_events + 8 * spikes + 4 * B * layer.n_neurons + dp.q.numel() * wbytes
        per_layer.append(dict(name=layer.name, updates=updates, spikes=spikes, lds_bytes=lds,
                              hbm_bytes=hbm, ms=float(launch_ms[i])))
        in_src, in_n = host[i]
    # Dominant kernel: the slowest layer.  Memory roof: HBM (the path does no MFMA work);
    # the LDS figure beside it is the on-chip roof the per-update traffic meets.
    dom = max(per_layer, key=lambda d: d["ms"])
    lds_gbs = dom["lds_bytes"] / (dom["ms"] * 1e-3) / 1e9
    hbm_gbs = dom["hbm_bytes"] / (dom["ms"] * 1e-3) / 1e9
    lds_frac, hbm_frac = lds_gbs / LDS_PEAK_GBS, hbm_gbs / HBM_PEAK_GBS
    roofline = {"bound": "hbm", "kernel": dom["name"], "launch_ms": round(dom["ms"], 4),
                "achieved": round(hbm_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(hbm_frac, 6), "traffic": measured_traffic(w.name, dom["name"]),
                "algorithmic_bytes": dom["hbm_bytes"],
                "lds": {"achieved": round(lds_gbs, 2), "peak": LDS_PEAK_GBS, "unit": "GB/s",
                        "frac": round(lds_frac, 5), "algorithmic_bytes": dom["lds_bytes"]},
                "layers": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                           for d in per_layer]}

    cpu = None
    bit_exact = None
    if not args.no_cpu:
        from oracle import oracle as O
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        specs = []
        for layer, p in zip(net.layers, w.params):
            if hasattr(layer, "oc"):
                g = dict(kind="conv", ic=layer.ic, h_in=layer.h_in, w_in=layer.w_in, oc=layer.oc,
                         k=layer.k, s=layer.s, p=layer.p, max_queue_len=layer.max_queue_len)
            else:
                g = dict(kind="fc", n_in=layer.n_in, n_out=layer.n_out)
            specs.append((g, dict(q=p.q, table=p.decay_table_int, v_th=p.v_th_int, f_a=p.f_a,
                                  f_V=p.f_V, i_V=p.i_V, round_mode=w.round_mode,
                                  overflow_mode=p.overflow_mode), layer.max_out_spikes))
        runs = []
        for _ in range(3):
            t_c = time.perf_counter()
            ref = O.network_forward(specs, *w.events, nthreads=threads)
            runs.append(time.perf_counter() - t_c)
        cpu_s = float(np.median(runs))
        # One thread on the first 64 streams (streams are independent and alike).
        sub = tuple(np.ascontiguousarray(a[:64]) for a in w.events)
        t_c = time.perf_counter()
        O.network_forward(specs, *sub, nthreads=1)
        one_s = time.perf_counter() - t_c
        cpu = {"value": round(n_events / cpu_s, 1), "unit": "input events/s", "cores": threads,
               "kind": "port",
               "sample": f"the full workload ({B} streams, {n_events} events, all three layers), "
                         f"oracle/salt_oracle.c -O3 with OpenMP over streams on {threads} host "
                         f"threads; median of 3 runs, {cpu_s:.3f} s",
               "single_thread_value": round(int(sub[2].sum()) / one_s, 1),
               "single_thread_sample": f"first 64 streams ({int(sub[2].sum())} events), 1 thread, "
                                       f"{one_s:.3f} s",
               "host_cpu": cpu_model()}
        bit_exact = True
        for o, r in zip(outs, ref):
            ok = (np.array_equal(o.n.cpu().numpy(), r["out_n"])
                  and np.array_equal(o.v_final.cpu().numpy(), r["v_final"])
                  and np.array_equal(o.stats[:, 0].cpu().numpy(), r["v_min"].min(axis=1))
                  and np.array_equal(o.stats[:, 1].cpu().numpy(), r["v_max"].max(axis=1)))
            cap = r["out_src"].shape[1]
            real = np.arange(cap)[None, :] < np.minimum(r["out_n"], cap)[:, None]
            for got, want in ((o.src.cpu().numpy(), r["out_src"]), (o.times.cpu().numpy(), r["out_times"])):
                ok = ok and np.array_equal(np.where(real, got[:, :cap], 0), np.where(real, want, 0))
            bit_exact = bit_exact and bool(ok)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "input events/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int32",
        "data": "synthetic",
        "config": {"workload": w.name, "streams": B, "padded_len": L, "input_events": n_events,
                   "layers": [l.name for l in net.layers],
                   "round_mode": w.round_mode,
                   "f_a": 10, "f_V": 0, "i_V": 24, "overflow": "wrap"},
        "bit_exact": bit_exact, "fits": bool(fits.all()),
        "end_to_end": {"ms": round(e2e_ms, 4), "value": round(n_events / (e2e_ms / 1000.0), 1),
                       "unit": "input events/s",
                       "what": "events from pinned host memory, one salt_network_forward call, "
                               "every layer's stream, registers and stats back to pinned host "
                               "memory (PCIe-inclusive), median of 5"},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if (bit_exact is not False and bool(fits.all())) else 1


if __name__ == "__main__":
    sys.exit(main())
