#!/usr/bin/env python3
"""Benchmark: integer event-by-event forward (salt_core/quant semantics) on one MI355X.

Default workload: the N-MNIST-shaped network of the benchmark configuration 3 (conv
2->16 5x5 s2 -> conv 16->32 3x3 s2 -> FC 1568->10, 1024 synthetic streams of ~4500
events); --config N runs configuration N instead.  A step = one forward of the whole
network over the batch, inputs resident in HBM, every layer's spike stream, final
registers and per-stream statistics written.

Prints one JSON line (the driver's contract).  value = layer-1 input events / second.
The step's output is checked bit for bit against the CPU oracle, whose timing on the
host cores is the cpu_baseline.

Roofline: three roofs for the dominant (slowest) layer kernel, the binding one named --
HBM (algorithmic bytes / launch time against 8 TB/s), LDS (algorithmic bytes against the
peak measured by --lds-peak, profiles/lds_peak.json) and VALU issue (the kernel's
SQ_INSTS_VALU per launch, profiles/sq_insts_<workload>.json, against one wave64 VALU
instruction per 4 cycles on each of the 1024 SIMDs at 2.4 GHz).

Other modes: --copy-calibration (the reference copy that scales FETCH_SIZE/WRITE_SIZE),
--lds-peak (the LDS probe), --digest DIR (rocprofv3 counter CSVs -> summary JSON).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "spiking-affine-lazy-training_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "input events/sec (batch, 1 MI355X) bit-exact vs salt_core/quant; % HBM/LDS roofline"
HBM_PEAK_GBS = 8000.0                     # MI355X HBM3E
CLOCK_GHZ = 2.4                           # MI355X peak engine clock
N_CU = 256
LDS_SPEC_GBS = N_CU * 128 * CLOCK_GHZ     # 128 B/clk per CU: the figure before measurement
VALU_PEAK_GINST = N_CU * 4 * CLOCK_GHZ / 4  # wave64 VALU instructions / ns: 4 SIMDs, 4 clk each
PROFILES = os.path.join(ROOT, "profiles")
LDS_PEAK_FILE = os.path.join(PROFILES, "lds_peak.json")
HBM_COPY_FILE = os.path.join(PROFILES, "hbm_copy.json")
TRAFFIC_FILE = os.path.join(PROFILES, "hbm_traffic_{workload}.json")
SQ_FILE = os.path.join(PROFILES, "sq_insts_{workload}.json")
COPY_BYTES = 1 << 30                      # --copy-calibration: bytes read (and written)
# Streams of the all-core CPU sample (None: the whole batch); every configuration's sample
# is about a second or two of oracle work per run on 16 host threads.
CPU_SAMPLE_STREAMS = {1: None, 2: None, 3: None, 4: None, 5: 512}
CPU_ONE_THREAD_STREAMS = {1: 1, 2: 32, 3: 64, 4: 4, 5: 8}


def _load_json(path):
    try:
        with open(path, encoding="utf-8") as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------ probes

def copy_calibration(out_path: str | None = None) -> int:
    """A plain device-to-device copy of COPY_BYTES, three times: the reference launch
    whose FETCH_SIZE / WRITE_SIZE readings scale the counters of the layer kernels.  Each
    copy is timed with HIP events on the copy's stream; the best of the three gives the
    measured copy bandwidth (bytes read + bytes written per second), reported beside the
    published 8 TB/s HBM peak (written to out_path when given)."""
    import torch
    torch.cuda.set_device(0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    ms = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        ms.append(e0.elapsed_time(e1))
    res = {"copy_bytes": COPY_BYTES, "launches": 3, "ms": [round(m, 4) for m in ms],
           "GB_per_s": round(2 * COPY_BYTES / (min(ms) * 1e-3) / 1e9, 1),
           "command": "python3 bench.py --copy-calibration"}
    line = json.dumps(res)
    print(line, flush=True)
    if out_path:
        with open(out_path, "w", encoding="utf-8") as f:
            f.write(line + "\n")
    return 0


def lds_peak(out_path: str | None) -> int:
    """LDS bandwidth of the device through libsalt_probe.so (salt_probe_lds): conflict-free
    32-, 64- and 128-bit reads and 32-bit writes, 4 work-groups of 256 threads per CU, each
    with 32 KB of LDS.  The peak used by the roofline is the largest read rate."""
    import ctypes

    import torch  # noqa: F401 -- loads the HIP runtime the probe library binds to
    torch.cuda.set_device(0)
    lib = ctypes.CDLL(os.path.join(PKG, "salt_amd", "libsalt_probe.so"))
    lib.salt_probe_lds.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                   ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
    lib.salt_probe_lds.restype = ctypes.c_int32
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = 4 * cus
    res = {"device": torch.cuda.get_device_name(0), "compute_units": cus, "blocks": blocks,
           "threads_per_block": 256, "lds_bytes_per_block": 32768, "accesses": {}}
    for kind, name, iters in ((0, "read_b32", 4000), (1, "read_b64", 2000), (2, "read_b128", 1000),
                              (3, "write_b32", 4000)):
        sec, nbytes = ctypes.c_double(0), ctypes.c_double(0)
        rc = lib.salt_probe_lds(kind, blocks, iters, ctypes.byref(sec), ctypes.byref(nbytes))
        if rc != 0:
            raise RuntimeError(f"salt_probe_lds({name}) failed: {rc}")
        gbs = nbytes.value / sec.value / 1e9
        res["accesses"][name] = {"iters": iters, "bytes": nbytes.value, "ms": sec.value * 1e3,
                                 "GB_per_s": round(gbs, 1),
                                 "bytes_per_clk_per_cu": round(gbs / (cus * CLOCK_GHZ), 1)}
        print(f"lds {name}: {gbs:.0f} GB/s", flush=True)
    reads = [v["GB_per_s"] for k, v in res["accesses"].items() if k.startswith("read")]
    res["peak_GB_per_s"] = max(reads)
    res["command"] = "python3 bench.py --lds-peak"
    line = json.dumps(res)
    print(line, flush=True)
    if out_path:
        with open(out_path, "w", encoding="utf-8") as f:
            f.write(line + "\n")
    return 0


LAYER_KERNELS = ("layer_kernel", "packed_kernel")   # one dispatch per layer
POST_KERNELS = ("compact_kernel",)                  # after their layer's kernel


def digest_counters(src_dir: str, config: int, kind: str, out_path: str, command: str) -> int:
    """rocprofv3 counter CSVs (every *counter_collection.csv under src_dir) of a bench.py run
    -> per-layer means per launch.  Layer kernels run in network order, so the i-th layer
    kernel dispatch (in dispatch-id order) is layer i mod n_layers; other profiled kernels
    (row-band list builds, fills, compactions) count towards the layer whose kernel follows
    them, compactions towards the one they follow.  kind "sq": SQ_* counters as they are;
    kind "traffic": the HBM bytes FETCH_SIZE x f + WRITE_SIZE x w with f, w read from the
    copy calibration files (copy_*.csv: the same counters for a COPY_BYTES device copy)."""
    from salt_amd import workloads as W
    names = [l.name for l in W.CONFIGS[config]().network.layers]
    rows = {}
    for path in sorted(glob.glob(os.path.join(src_dir, "**", "*counter_collection.csv"), recursive=True)):
        is_copy = "copy" in os.path.relpath(path, src_dir)  # the calibration run's files
        with open(path, newline="", encoding="utf-8") as f:
            for r in csv.DictReader(f):
                key = ("copy" if is_copy else "run", path, int(r["Dispatch_Id"]))
                v = rows.setdefault(key, {"kernel": r["Kernel_Name"]})
                v[r["Counter_Name"]] = v.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    runs, copies = {}, {}
    for (what, path, did), v in sorted(rows.items()):
        (copies if what == "copy" else runs).setdefault(path, []).append(v)
    per_launch: dict[str, list] = {n: [] for n in names}   # summed counters per layer launch
    per_kernel: dict[str, dict[str, list]] = {}
    kernels: dict[str, list] = {n: [] for n in names}
    for path, disp in runs.items():
        i_layer, pending, last = 0, [], None
        for v in disp:
            k = v["kernel"]
            short = k[:120]
            for c, x in v.items():
                if c != "kernel":
                    per_kernel.setdefault(short, {}).setdefault(c, []).append(x)
            if any(t in k for t in LAYER_KERNELS):
                name = names[i_layer % len(names)]
                i_layer += 1
                launch = {}
                for u in pending + [v]:
                    for c, x in u.items():
                        if c != "kernel":
                            launch[c] = launch.get(c, 0.0) + x
                per_launch[name].append(launch)
                for u in pending + [v]:
                    if u["kernel"][:120] not in kernels[name]:
                        kernels[name].append(u["kernel"][:120])
                pending, last = [], name
            elif any(t in k for t in POST_KERNELS) and last is not None and per_launch[last]:
                for c, x in v.items():
                    if c != "kernel":
                        per_launch[last][-1][c] = per_launch[last][-1].get(c, 0.0) + x
                if short not in kernels[last]:
                    kernels[last].append(short)
            else:
                pending.append(v)
    # each counter's mean over the launches that carry it (one pass per counter or group)
    means = {}
    for n, L in per_launch.items():
        cs = sorted({c for d in L for c in d})
        means[n] = {c: sum(d[c] for d in L if c in d) / sum(1 for d in L if c in d) for c in cs}
    kmeans = {k: {c: sum(x) / len(x) for c, x in d.items()} for k, d in per_kernel.items()}
    out = {"what": f"per-launch means of rocprofv3 counters, layers of {W.CONFIGS[config]().name} "
                   "(each layer's kernels summed), and per-dispatch means per kernel",
           "command": command, "kernels": kernels, "per_layer": means, "per_kernel": kmeans}
    if kind == "traffic":
        cal = {}
        for disp in copies.values():
            for v in disp:
                if "copy" not in v["kernel"].lower():
                    continue
                for c in ("FETCH_SIZE", "WRITE_SIZE"):
                    if c in v:
                        cal.setdefault(c, []).append(v[c])
        fac = {c: COPY_BYTES / (max(x) * 1024.0) for c, x in cal.items() if x}
        out["copy_calibration"] = {"bytes": COPY_BYTES, "factor": fac}

        def hbm(m):
            return round(m.get("FETCH_SIZE", 0) * 1024 * fac.get("FETCH_SIZE", 1.0)
                         + m.get("WRITE_SIZE", 0) * 1024 * fac.get("WRITE_SIZE", 1.0))
        out["per_launch_bytes"] = {n: hbm(m) for n, m in means.items()}
        out["per_kernel_bytes"] = {k: hbm(m) for k, m in kmeans.items()}
    with open(out_path, "w", encoding="utf-8") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out)[:2000], flush=True)
    return 0


# ------------------------------------------------------------------ host facts

def host_cpu_facts() -> dict:
    """CPU model and the cores this process may use."""
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if model == "unknown":
        try:
            with open("/proc/cpuinfo", encoding="utf-8") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"model": model, "os_cpu_count": os.cpu_count(), "affinity": affinity,
            "OMP_NUM_THREADS": omp}


def cpu_threads(facts: dict, requested: int) -> tuple[int, str]:
    """All cores this process may use: the affinity set, within the host's per-GPU share
    when the environment states one (OMP_NUM_THREADS)."""
    if requested > 0:
        return requested, "--cpu-threads"
    omp = facts["OMP_NUM_THREADS"]
    if omp and omp.isdigit() and int(omp) > 0 and int(omp) < facts["affinity"]:
        return int(omp), (f"OMP_NUM_THREADS={omp}: the host's CPU share for this GPU "
                          f"(affinity set {facts['affinity']} of {facts['os_cpu_count']} CPUs)")
    return facts["affinity"], f"every CPU of the affinity set ({facts['affinity']} of {facts['os_cpu_count']})"


# ------------------------------------------------------------------ workload facts

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
    return (per_event * real).sum(axis=1, dtype=np.int64)


def oracle_specs(net, params, round_mode):
    specs = []
    for layer, p in zip(net.layers, params):
        if hasattr(layer, "oc"):
            g = dict(kind="conv", ic=layer.ic, h_in=layer.h_in, w_in=layer.w_in, oc=layer.oc,
                     k=layer.k, s=layer.s, p=layer.p, max_queue_len=layer.max_queue_len)
        else:
            g = dict(kind="fc", n_in=layer.n_in, n_out=layer.n_out)
        specs.append((g, dict(q=p.q, table=p.decay_table_int, v_th=p.v_th_int, f_a=p.f_a,
                              f_V=p.f_V, i_V=p.i_V, round_mode=round_mode,
                              overflow_mode=p.overflow_mode), layer.max_out_spikes))
    return specs


def oracle_forward(O, specs, events, threads):
    """The oracle over a batch: one layer in hash mode (no B x cap output buffers), or the
    whole chain with full streams (each layer's stream feeds the next)."""
    t, s, n = events
    if len(specs) == 1:
        g, p, cap = specs[0]
        return [O.layer_forward(g, p, t, s, n, cap, nthreads=threads, hashed=True)]
    return O.network_forward(specs, t, s, n, nthreads=threads)


def end_to_end(runner, w, dev, reps=5):
    """Host -> device -> host: the events copied from pinned host memory, the whole network
    in one salt_network_forward call, then every layer's spike count; each layer's streams
    are copied back up to the batch's largest count (the rest is padding), with the final
    registers and stats.  The PCIe-inclusive time of one batch (median of reps)."""
    import numpy as np
    import torch
    from salt_amd.stream import EventStream, unit_gain
    t_h = torch.from_numpy(np.ascontiguousarray(w.events.event_times, dtype=np.float32)).pin_memory()
    s_h = torch.from_numpy(np.ascontiguousarray(w.events.source_idx, dtype=np.int32)).pin_memory()
    n_h = torch.from_numpy(np.ascontiguousarray(w.events.n_real_events, dtype=np.int32)).pin_memory()
    n_layers = len(w.network.layers)
    counts_h = torch.empty((n_layers, n_h.shape[0]), dtype=torch.int32, pin_memory=True)
    times = []
    moved = 0
    for _ in range(reps + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        t_d = t_h.to(dev, non_blocking=True)
        stream = EventStream(event_times=t_d, event_source_idx=s_h.to(dev, non_blocking=True),
                             event_gain=unit_gain(t_d), n_real_events=n_h.to(dev, non_blocking=True))
        outs = runner.run(stream)
        for i, o in enumerate(outs):
            counts_h[i].copy_(o.n, non_blocking=True)
        torch.cuda.synchronize()
        moved = 0
        host = []
        for i, o in enumerate(outs):
            m = min(int(counts_h[i].max()), o.times.shape[1])
            for x in ((o.times[:, :m], o.src[:, :m]) if m else ()) + (o.v_final, o.stats):
                h = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
                h.copy_(x, non_blocking=True)
                host.append(h)
                moved += h.numel() * h.element_size()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return float(np.median(times[1:])) * 1000.0, moved


# ------------------------------------------------------------------ main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, help="benchmark configuration 1..5")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle threads (0: the CPUs this process may use)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and the check")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the reference copy used to scale HBM traffic counters")
    ap.add_argument("--lds-peak", action="store_true", help="only run the LDS bandwidth probe")
    ap.add_argument("--out", default=None,
                    help="--lds-peak / --copy-calibration / --digest: file to write")
    ap.add_argument("--digest", default=None, metavar="DIR",
                    help="summarise the rocprofv3 counter CSVs under DIR (no GPU)")
    ap.add_argument("--digest-kind", default="sq", choices=("sq", "traffic"))
    ap.add_argument("--digest-command", default="", help="the profiling command, recorded")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.out)
    if args.lds_peak:
        return lds_peak(args.out)
    if args.digest:
        return digest_counters(args.digest, args.config, args.digest_kind, args.out,
                               args.digest_command)
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
    from salt_amd.stream import stream_hash

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    w = W.CONFIGS[args.config]()
    net = w.network
    runner = NetworkRunner(net, w.params, w.round_mode, dev)
    stream = net.input_stream(w.events, device=dev)
    n_events = int(np.minimum(w.events.n_real_events, w.events.event_times.shape[1]).sum())
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

    e2e_ms, e2e_bytes = end_to_end(runner, w, dev)

    # Algorithmic traffic of each layer (per launch): LDS = updates x (4 + 4 + weight bytes);
    # HBM = 8 B per input event + 8 B per spike + 4 B per final register + weights, + 8 B per
    # pad entry of a layer whose output stream is filled to its capacity (the last layer's,
    # as the reference's EventStream of max_out_spikes entries is).
    host = [(o.src.cpu().numpy(), o.n.cpu().numpy()) for o in outs]
    in_src, in_n = w.events.source_idx, w.events.n_real_events
    per_layer = []
    for i, (layer, dp) in enumerate(zip(net.layers, runner.dev_params)):
        wbytes = dp.q_bits // 8
        n_eff = np.minimum(in_n, in_src.shape[1])
        n_in_events = int(n_eff.sum())
        if hasattr(layer, "oc"):
            updates = int(conv_update_counts(layer, in_src, n_eff).sum())
        else:
            updates = n_in_events * layer.n_out
        spikes = int(host[i][1].sum())
        pads = int(np.maximum(layer.max_out_spikes - host[i][1], 0).sum()) if i == n_layers - 1 else 0
        lds = updates * (8 + wbytes)
        hbm = 8 * n_in_events + 8 * spikes + 8 * pads + 4 * B * layer.n_neurons + dp.q.numel() * wbytes
        per_layer.append(dict(name=layer.name, updates=updates, spikes=spikes, pad_entries=pads,
                              lds_bytes=lds, hbm_bytes=hbm, ms=float(launch_ms[i])))
        in_src, in_n = host[i]

    # Dominant kernel: the slowest layer; its three roofs, the binding one named.
    dom = max(per_layer, key=lambda d: d["ms"])
    sec = dom["ms"] * 1e-3
    lds_prof = _load_json(LDS_PEAK_FILE)
    hbm_copy = _load_json(HBM_COPY_FILE)
    lds_peak_gbs = lds_prof["peak_GB_per_s"] if lds_prof else LDS_SPEC_GBS
    traffic = _load_json(TRAFFIC_FILE.format(workload=w.name))
    sq = _load_json(SQ_FILE.format(workload=w.name))
    roofs = {
        "hbm": {"achieved": round(dom["hbm_bytes"] / sec / 1e9, 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "algorithmic_bytes": dom["hbm_bytes"],
                "measured_copy_GB_per_s": (hbm_copy or {}).get("GB_per_s"),
                "measured_copy_source": "profiles/hbm_copy.json (bench.py --copy-calibration)"},
        "lds": {"achieved": round(dom["lds_bytes"] / sec / 1e9, 2), "peak": round(lds_peak_gbs, 1),
                "unit": "GB/s", "algorithmic_bytes": dom["lds_bytes"],
                "peak_source": "profiles/lds_peak.json (bench.py --lds-peak)" if lds_prof
                else "assumed: 128 B/clk per CU"},
    }
    valu = sq and sq.get("per_layer", {}).get(dom["name"], {}).get("SQ_INSTS_VALU")
    if valu:
        roofs["valu"] = {"achieved": round(valu / sec / 1e9, 2), "peak": VALU_PEAK_GINST,
                         "unit": "G wave64 VALU instructions/s", "instructions": valu,
                         "source": f"profiles/sq_insts_{w.name}.json (SQ_INSTS_VALU per launch)"}
    for r in roofs.values():
        r["frac"] = round(r["achieved"] / r["peak"], 5)
    bound = max(roofs, key=lambda k: roofs[k]["frac"])
    traffic_bytes = traffic and traffic.get("per_launch_bytes", {}).get(dom["name"])
    roofline = {"bound": bound, "kernel": dom["name"], "launch_ms": round(dom["ms"], 4),
                "achieved": roofs[bound]["achieved"], "peak": roofs[bound]["peak"],
                "unit": roofs[bound]["unit"], "frac": roofs[bound]["frac"],
                "traffic": traffic_bytes, "algorithmic_hbm_bytes": dom["hbm_bytes"],
                "roofs": roofs,
                "layers": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                           for d in per_layer]}

    cpu = None
    bit_exact = None
    if not args.no_cpu:
        from oracle import oracle as O
        facts = host_cpu_facts()
        threads, why = cpu_threads(facts, args.cpu_threads)
        specs = oracle_specs(net, w.params, w.round_mode)
        ns = CPU_SAMPLE_STREAMS.get(args.config) or B
        sample = tuple(np.ascontiguousarray(a[:ns]) for a in w.events)
        sample_events = int(np.minimum(sample[2], L).sum())
        runs = []
        ref = None
        for r in range(7):  # 2 warm-ups, 5 timed
            t_c = time.perf_counter()
            ref = oracle_forward(O, specs, sample, threads)
            if r >= 2:
                runs.append(time.perf_counter() - t_c)
        cpu_s = float(np.median(runs))
        n1 = min(B, CPU_ONE_THREAD_STREAMS.get(args.config, 64))
        sub1 = tuple(np.ascontiguousarray(a[:n1]) for a in w.events)
        one = []
        for r in range(3):
            t_c = time.perf_counter()
            oracle_forward(O, specs, sub1, 1)
            if r >= 1:
                one.append(time.perf_counter() - t_c)
        one_s = float(np.median(one))
        cpu = {"value": round(sample_events / cpu_s, 1), "unit": "input events/s", "cores": threads,
               "kind": "port",
               "sample": (f"{'the full workload' if ns >= B else f'the first {ns} of {B} streams'} "
                          f"({sample_events} input events, all {n_layers} layer(s)); "
                          f"oracle/salt_oracle.c -O3 -march=x86-64-v3, OpenMP over streams on "
                          f"{threads} threads; median of 5 runs after 2 warm-ups, {cpu_s:.3f} s"),
               "threads_reason": why, "host_cpu": facts["model"], "os_cpu_count": facts["os_cpu_count"],
               "affinity_cpus": facts["affinity"], "OMP_NUM_THREADS": facts["OMP_NUM_THREADS"],
               "single_thread_value": round(int(np.minimum(sub1[2], L).sum()) / one_s, 1),
               "single_thread_sample": f"first {n1} stream(s), 1 thread, median of 2 after 1 warm-up, "
                                       f"{one_s:.3f} s"}
        # Bit-exactness of the step's output: the whole batch (the oracle again when the
        # timed sample was a subset).
        if ns < B:
            ref = oracle_forward(O, specs, w.events, threads)
        bit_exact = True
        for o, r in zip(outs, ref):
            ok = (np.array_equal(o.n.cpu().numpy(), r["out_n"])
                  and np.array_equal(o.v_final.cpu().numpy(), r["v_final"])
                  and np.array_equal(o.stats[:, 0].cpu().numpy(), r["v_min"].min(axis=1))
                  and np.array_equal(o.stats[:, 1].cpu().numpy(), r["v_max"].max(axis=1)))
            if "out_hash" in r:
                from salt_amd.stream import EventStream, unit_gain
                st = EventStream(o.times, o.src, unit_gain(o.times), o.n)
                ok = ok and np.array_equal(stream_hash(st).cpu().numpy().view(np.uint64), r["out_hash"])
            else:
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
                   "f_a": W.F_A, "f_V": W.F_V, "i_V": W.I_V, "overflow": "wrap"},
        "bit_exact": bit_exact, "fits": bool(fits.all()),
        "end_to_end": {"ms": round(e2e_ms, 4), "value": round(n_events / (e2e_ms / 1000.0), 1),
                       "unit": "input events/s", "bytes_back": e2e_bytes,
                       "what": "events from pinned host memory, one salt_network_forward call, "
                               "the spike counts, then every layer's streams up to the batch's "
                               "largest count, registers and stats back to pinned host memory "
                               "(PCIe-inclusive), median of 5"},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if (bit_exact is not False and bool(fits.all())) else 1


if __name__ == "__main__":
    sys.exit(main())
