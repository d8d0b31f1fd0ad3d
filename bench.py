"""Benchmark of the MI355X token sampler.

One step = one launch of the sampler over one [B=64, V=151936] fp32 batch:
penalties from 2048-id histories (rep 1.1, frequency 0.5, presence 0.3),
temperature 0.7, top-k 50, softmax and the draw. Inputs are seeded synthetic
data, resident in HBM before timing. Eight distinct input sets (315 MB, more
than the 256 MB Infinity Cache) rotate so the kernel streams from HBM.

The launches of one rotation are captured into a HIP graph (torch.cuda.CUDAGraph)
and replayed; HIP events on the launch stream bracket the K timed steps. A
second graph of the same launches with only the pass over the logits (the
library's STREAM_ONLY diagnostics flag), timed the same way, gives the stream
kernel's own duration (the merge takes the rest of the step); the roofline
figure is the stream kernel's algorithmic bytes over that duration.
Prints one JSON line (see `main`). The CPU baseline is the reference's own
sampler (oracle/_ref, compiled from its sources) or, where that was not
built, the CPU restatement, timed on this host's cores on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sampled rows/sec at B=64,V=151936 fp32; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0
N_SETS = 8


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 4, 5])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=1.5,
                    help="wall seconds of the CPU baseline sample (all threads)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run 3 device-to-device copies of this many MiB (a known-size "
                         "kernel that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def cpu_baseline(wl, seconds: float):
    """The reference sampler on this host, rows split over the host's cores."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O  # the checker / baseline, never the product
    threads = max(1, min(16, os.cpu_count() or 1))
    kind = "reference" if O.ref_available() else "port"
    x0 = wl.logits_f32()
    hist = wl.hist if wl.hist is not None else np.zeros((wl.rows, 1), np.int32)
    hl = wl.hist_len if wl.hist_len is not None else np.zeros(wl.rows, np.int64)
    seeds = np.arange(wl.rows, dtype=np.uint64) + 1
    timed, rows, passes = 0.0, 0, 0
    while timed < seconds or passes < 2:
        x = x0.copy()
        t0 = time.perf_counter()
        if kind == "reference":
            O.ref_sample_batch(x, wl.params, hist, hl, seeds, nthreads=threads)
        else:
            O.sample_batch(x, wl.params, hist, hl, wl.mask, wl.u, nthreads=threads)
        timed += time.perf_counter() - t0
        rows += wl.rows
        passes += 1
    return {"value": rows / timed, "unit": "rows/s", "cores": threads, "kind": kind,
            "sample": f"{passes} passes over the {wl.rows}-row {wl.name} batch "
                      f"({rows} rows, {timed:.2f} s wall on {threads} threads)"}


def traffic_from_profiles(cfg: int):
    f = ROOT / "profiles" / f"k_stream_cfg{cfg}_traffic.json"
    if f.exists():
        try:
            return json.loads(f.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(rows shard across GPUs with no exchange: the figure is N x the 1-GPU value).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    wlm, hs = pkg.workloads, pkg.hsamp
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    sets = [wlm.config(args.config, seed=100 + i) for i in range(N_SETS)]
    wl0 = sets[0]
    B, V = wl0.rows, wl0.vocab
    to_dev = []
    for w in sets:
        if w.dtype == "f32":
            x = torch.from_numpy(w.logits).to(dev)
        else:
            x = torch.from_numpy(w.logits.view(np.int16)).to(dev).view(torch.bfloat16)
        u = torch.from_numpy(w.u).to(dev)
        h = None if w.hist is None else torch.from_numpy(w.hist).to(dev)
        m = None if w.mask is None else torch.from_numpy(w.mask.view(np.int32)).to(dev)
        to_dev.append((x, u, h, m))
    sampler = hs.Sampler(0, max_rows=max(B, 64), max_vocab=V)
    stream = torch.cuda.Stream(dev)
    outs = [{"token": torch.empty(B, dtype=torch.int32, device=dev),
             "row_flags": torch.empty(B, dtype=torch.int32, device=dev)} for _ in sets]

    def launch(i, s):
        x, u, h, m = to_dev[i]
        sampler.run(x, sets[i].params, u, hist=h, hist_len=sets[i].hist_len, mask=m,
                    outputs=outs[i], stream=s)

    with torch.cuda.stream(stream):
        for i in range(N_SETS):          # uncaptured first run: uploads knobs, sizes scratch
            launch(i, stream)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(N_SETS):
            launch(i, stream)
    stream.synchronize()

    reps_w = max(1, args.warmup // N_SETS)
    reps = max(1, args.steps // N_SETS)
    steps = reps * N_SETS
    with torch.cuda.stream(stream):
        for _ in range(reps_w):
            graph.replay()
    stream.synchronize()
    torch.cuda.synchronize()
    t0e = torch.cuda.Event(enable_timing=True)
    t1e = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    with torch.cuda.stream(stream):
        t0e.record(stream)
        for _ in range(reps):
            graph.replay()
        t1e.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_total = t0e.elapsed_time(t1e)
    ms_step = ms_total / steps

    # Per-kernel split, live: a second graph holds the same launches with only
    # the pass over the logits (k_stream; the library's STREAM_ONLY
    # diagnostics flag), replayed between events like the full step; the
    # per-row merge (k_pick or k_merge) takes the rest of the step.
    def launch_stream_only(i, s):
        x, u, h, m = to_dev[i]
        sampler.run(x, sets[i].params, u, hist=h, hist_len=sets[i].hist_len, mask=m,
                    outputs=outs[i], stream=s, stream_only=True)

    sgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(sgraph, stream=stream):
        for i in range(N_SETS):
            launch_stream_only(i, stream)
    stream.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(reps_w):
            sgraph.replay()
    stream.synchronize()
    s0e = torch.cuda.Event(enable_timing=True)
    s1e = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        s0e.record(stream)
        for _ in range(reps):
            sgraph.replay()
        s1e.record(stream)
    stream.synchronize()
    n_split = reps * N_SETS
    stream_ms = s0e.elapsed_time(s1e) / n_split
    merge_ms = ms_step - stream_ms
    del sgraph

    # The replayed outputs are the real ones: spot-check them against an
    # uncaptured launch of the same inputs.
    ref_tok = [o["token"].clone() for o in outs]
    with torch.cuda.stream(stream):
        for i in range(N_SETS):
            launch(i, stream)
    stream.synchronize()
    for i in range(N_SETS):
        if not torch.equal(ref_tok[i], outs[i]["token"]):
            raise SystemExit("graph replay and direct launch disagree")

    algo_bytes = wl0.algorithmic_bytes()
    # the per-row merge kernel these batches take: k_pick after exact lists
    # (every row samples with top-k <= 64), k_merge for the general kernels
    exact_on = os.environ.get("ULTIMA_HSAMP_EXACT", "1")[:1] != "0"
    merge_name = "k_pick" if (exact_on and args.config in (1, 2, 4)) else "k_merge"
    achieved = algo_bytes / (stream_ms * 1e-3) / 1e9   # k_stream: the kernel that reads the logits
    line = {
        "metric": METRIC,
        "value": B / (ms_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * N_SETS,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if wl0.dtype == "f32" else "bf16",
        "data": "synthetic (seeded SplitMix64/Box-Muller logits and histories, 8 rotating sets)",
        "config": {"workload": f"cfg{args.config}: B={B} V={V} {wl0.dtype} "
                               + ("hist 2048 rep 1.1 freq .5 pres .3 T .7 top-k 50"
                                  if args.config == 2 else wl0.name),
                   "rows": B, "vocab": V, "input_sets": N_SETS,
                   "bytes_per_step": algo_bytes, "wall_s": round(wall, 4),
                   "kernel_us": {"k_stream": round(stream_ms * 1e3, 3), merge_name: round(merge_ms * 1e3, 3),
                                 "launches_timed": n_split},
                   "step_hbm_gbs": round(algo_bytes / (ms_step * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBS, "traffic": traffic_from_profiles(args.config),
                     "kernel": "k_stream", "algorithmic_bytes_per_launch": algo_bytes},
        "cpu_baseline": None,
    }
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["config"]["copy_probe_bytes"] = n * 4
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(wl0, args.cpu_seconds)
    sampler.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
