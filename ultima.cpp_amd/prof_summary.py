"""Summarise rocprofv3 runs of bench.py into the text kept under profiles/.

Inputs are three rocprofv3 output folders of the same bench command:
  --stats  a `--kernel-trace --stats` run (per-kernel average durations)
  --fetch  a `--pmc FETCH_SIZE` run, --write a `--pmc WRITE_SIZE` run
           (KiB per dispatch), both with `bench.py --copy-probe-mib M`: the
           M MiB device copy they end with calibrates each counter (bytes it
           must have moved / what the counter reported for it).

Writes <out>/<kernels>_<tag>_profile.md (kernel durations, traffic per
kernel, the commands) and, for the workload's dominant kernel (the one that
reads the logits, or the lm-head matvec), <out>/<kernel>_<tag>_traffic.json,
which bench.py reads for roofline.traffic. <tag> is cfg1 .. cfg5, head or
head_<type>, or cli (bench.py --workload cli: the step's kernels k_fs_max,
k_fs_exp and k_full taken together as its traffic).

    python3 ultima.cpp_amd/prof_summary.py --config 2 --stats DIR --fetch DIR --write DIR \
        --bench DIR/stats_bench.json --copy-mib 512 --out profiles --command "..."
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
from collections import defaultdict
from pathlib import Path

COPY_KERNEL = "__amd_rocclr_copyBuffer"
STREAM_KERNEL = {"cfg1": "k_stream", "cfg2": "k_stream", "cfg3": "k_full", "cfg4": "k_stream", "cfg5": "k_stream",
                 "head": "k_head_gemv", "cli": "k_full"}


def short(name: str) -> str:
    """'void hsamp::k_stream<0, true, ...>(hsamp::StreamArgs)' -> 'k_stream<0, true, ...>'"""
    n = name
    for p in ("void ", "hsamp::", "(anonymous namespace)::"):
        n = n.replace(p, "")
    return n.split("(")[0]


def one_csv(folder: Path, suffix: str) -> Path:
    files = sorted(folder.rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {folder}")
    return files[0]


def kernel_stats(folder: Path) -> list[dict]:
    rows = list(csv.DictReader(one_csv(folder, "kernel_stats.csv").open()))
    return [r for r in rows if "hsamp::" in r["Name"]]


def counter(folder: Path) -> dict[str, list[float]]:
    per = defaultdict(list)
    for r in csv.DictReader(one_csv(folder, "counter_collection.csv").open()):
        per[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return per


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", required=True,
                    help="1-5 (a sampler configuration), head (the bf16 head), head_<type> (bench.py --head-dtype) "
                         "or cli (bench.py --workload cli)")
    ap.add_argument("--stats", type=Path, required=True)
    ap.add_argument("--fetch", type=Path, required=True)
    ap.add_argument("--write", type=Path, required=True)
    ap.add_argument("--bench", type=Path, required=True, help="the bench JSON line of the stats run")
    ap.add_argument("--copy-mib", type=int, required=True)
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--command", action="append", default=[], help="a command that made the inputs (repeatable)")
    a = ap.parse_args()

    bench = json.loads(a.bench.read_text().strip().splitlines()[-1])
    algo = int(bench["config"]["bytes_per_step"])
    stats = kernel_stats(a.stats)
    fetch, write = counter(a.fetch), counter(a.write)
    copy_kib = a.copy_mib * 1024.0
    f_copy, w_copy = max(fetch.get(COPY_KERNEL, [0.0])), max(write.get(COPY_KERNEL, [0.0]))
    if f_copy <= 0 or w_copy <= 0:
        raise SystemExit("the calibration copy is missing from the counter runs")
    fs, ws = copy_kib / f_copy, copy_kib / w_copy

    table = []
    for r in stats:
        name = r["Name"]
        f = statistics.median(fetch[name]) if fetch.get(name) else None
        w = statistics.median(write[name]) if write.get(name) else None
        hbm = None if f is None or w is None else (f * fs + w * ws) * 1024.0
        table.append((short(name), int(r["Calls"]), float(r["AverageNs"]) / 1000.0, f, w, hbm))

    tag = a.config if a.config.startswith("head") or a.config == "cli" else f"cfg{int(a.config)}"
    # head_<type>: a quantised head (k_head_q) or a dense one (k_head_gemv)
    sk = STREAM_KERNEL.get(tag, "k_head_gemv" if tag in ("head_f32", "head_bf16") else "k_head_q")
    main_row = next((t for t in table if t[0].startswith(sk + "<") and t[5] is not None), None)
    if tag == "cli":
        # the step's four kernels, each launched once per step
        parts = [t for t in table if t[0].split("<")[0] in ("k_fs_max", "k_fs_exp", "k_full")]
        if parts and all(t[5] is not None for t in parts):
            main_row = ("k_fs_* + k_full", min(t[1] for t in parts), sum(t[2] for t in parts),
                        sum(t[3] for t in parts), sum(t[4] for t in parts), sum(t[5] for t in parts))
    wl = bench["config"]["workload"]
    lines = [f"# rocprofv3 profile, workload {wl}", ""]
    lines += ["Commands (from the repository root on the GPU box):", ""]
    lines += [f"    {c}" for c in a.command] + [""]
    lines += [f"Calibration: the {a.copy_mib} MiB device copy (`{COPY_KERNEL}`) read as "
              f"{f_copy:.0f} KiB by FETCH_SIZE (scale {fs:.3f}) and {w_copy:.0f} KiB by WRITE_SIZE "
              f"(scale {ws:.3f}). Counter figures are medians over the dispatches; durations are "
              "rocprofv3's averages over every dispatch of the stats run (graph replays of the full "
              "step and of the stream kernel alone, read probes and uncaptured calls).", ""]
    lines += ["| kernel | dispatches | avg us | FETCH KiB | WRITE KiB | HBM bytes (scaled) | x algorithmic |",
              "|---|---|---|---|---|---|---|"]
    for n, c, us, f, w, hbm in table:
        ratio = "" if hbm is None else f"{hbm / algo:.3f}"
        lines.append(f"| `{n}` | {c} | {us:.2f} | {'' if f is None else f'{f:.1f}'} | "
                     f"{'' if w is None else f'{w:.1f}'} | {'' if hbm is None else f'{hbm:.0f}'} | {ratio} |")
    what = ("the head's weights, the hidden states, the norm scale, the normed rows and the logits, "
            "each once" if tag.startswith("head") else "each logit, history id and mask word read once, u and the token")
    if main_row is not None and tag == "cli":
        lines += [f"The step's kernels together: {main_row[5]:.0f} HBM bytes per step, "
                  f"{main_row[5] / algo:.3f} x algorithmic, {main_row[2]:.2f} us of kernel time.", ""]
    lines += ["", f"Algorithmic bytes per step: {algo} ({what}).", ""]
    lines += ["Bench line of the stats run (timings perturbed by the tracer):", "",
              "    " + json.dumps({k: bench[k] for k in ("value", "ms_per_step")} |
                                    {"kernel_us": bench["config"].get("kernel_us"),
                                     "ceiling_us": (bench.get("roofline") or {}).get("ceiling_us")}), ""]
    a.out.mkdir(parents=True, exist_ok=True)
    kernels = []
    for n, *_ in table:
        base = n.split("<")[0]
        if base not in kernels and base != "k_read_probe":
            kernels.append(base)
    md = a.out / f"{'_'.join(sorted(kernels, key=lambda k: (k != sk, k)))}_{tag}_profile.md"
    md.write_text("\n".join(lines))
    if main_row is not None:
        js = {"kernel": sk, "workload": tag, "kernel_name": main_row[0],
              "fetch_kib": main_row[3], "write_kib": main_row[4], "fetch_scale": fs, "write_scale": ws,
              "hbm_bytes_per_launch": main_row[5], "algorithmic_bytes": algo, "avg_us": main_row[2],
              "source": f"profiles/{md.name}"}
        (a.out / f"{sk}_{tag}_traffic.json").write_text(json.dumps(js, indent=1) + "\n")
    print(md)


if __name__ == "__main__":
    main()
