"""rocprofv3 dispatch durations of bench.py's own timed kernel runs: pairs the kernel trace of a
profiled bench.py run (`rocprofv3 --kernel-trace -f csv`) with the ordered run list bench.py
writes with --trace-labels, so that each of bench.py's HIP-event figures has the profiler's
duration of exactly the same launches beside it.

    rocprofv3 --kernel-trace --stats -f csv -d OUT/bk -o bk -- \\
        python3 bench.py --section kernels,fused_gemm --path per-step --trace-labels OUT/labels.json
    python julia-cuda_amd/kernel_trace.py OUT/bk OUT/labels.json --out profiles/bench_kernels_rocprof.json

A label's run is the next stretch of consecutive dispatches whose kernel names contain the
label's instance, at least warm-up + timed long; its timed launches are the last `timed` of the
stretch. Prints a table (label, kernel, launches, average / median / min / max us) and writes
{"runs": {label: {...}}} for bench.py.
"""

import argparse
import csv
import glob
import json
import os
import statistics


def dispatches(path):
    files = [path] if os.path.isfile(path) else sorted(
        glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no kernel_trace CSV under {path}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3) for r in rows]


def stretches(ds, part):
    """[(first index, [names], [durations])] of maximal runs of consecutive dispatches whose
    kernel names contain `part` (one instance, or several: the attention step alternates the
    global and window layers' kernels)."""
    out, cur = [], None
    for i, (name, us) in enumerate(ds):
        if part in name:
            if cur is None:
                cur = (i, [], [])
                out.append(cur)
            cur[1].append(name)
            cur[2].append(us)
        else:
            cur = None
    return out


def pair(ds, labels):
    runs, at = {}, 0
    for lab in labels:
        need = lab["warmup"] + lab["timed"]
        found = [s for s in stretches(ds, lab["kernel"]) if s[0] >= at and len(s[2]) >= need]
        if not found:
            raise SystemExit(f"no run of {lab['kernel']} ({need} launches) for {lab['label']}")
        i0, names, durs = found[0]
        us = durs[-lab["timed"]:]
        names = sorted(set(names[-lab["timed"]:]))
        runs[lab["label"]] = {"kernel": lab["kernel"], "name": " + ".join(names), "launches": len(us),
                              "avg_us": round(statistics.mean(us), 3),
                              "median_us": round(statistics.median(us), 3),
                              "min_us": round(min(us), 3), "max_us": round(max(us), 3)}
        at = i0 + len(durs)
    return runs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace", help="rocprofv3 output directory or kernel_trace CSV")
    ap.add_argument("labels", help="bench.py --trace-labels output")
    ap.add_argument("--out")
    args = ap.parse_args()
    with open(args.labels) as fh:
        labels = json.load(fh)
    runs = pair(dispatches(args.trace), labels)
    print("| run | kernel | launches | avg us | median us | min us | max us |")
    print("|---|---|---:|---:|---:|---:|---:|")
    for k, r in runs.items():
        print(f"| {k} | `{r['name']}` | {r['launches']} | {r['avg_us']} | {r['median_us']} | "
              f"{r['min_us']} | {r['max_us']} |")
    if args.out:
        with open(args.out, "w") as fh:
            json.dump({"runs": runs}, fh, indent=1)
            fh.write("\n")


if __name__ == "__main__":
    main()
