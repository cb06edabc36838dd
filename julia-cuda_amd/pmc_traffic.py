"""HBM traffic per dispatch of one kernel from two rocprofv3 counter runs (FETCH_SIZE, then
WRITE_SIZE, in KiB per dispatch), each scaled by what the same counter reads for the library's
plain copy kernel (stream_copy_kernel, `--copy-bytes` read and written per dispatch) in the same
run. Run kernel_bench.py under each pass:

    rocprofv3 --pmc FETCH_SIZE -f csv -d OUT/fetch -o pmc -- python3 julia-cuda_amd/kernel_bench.py --step qkv
    rocprofv3 --pmc WRITE_SIZE -f csv -d OUT/write -o pmc -- python3 julia-cuda_amd/kernel_bench.py --step qkv
    python julia-cuda_amd/pmc_traffic.py --fetch OUT/fetch --write OUT/write \\
        --kernel gemm_latILi32ELi20E --copy-bytes 67108864 --algorithmic 5451488

Prints (and with --out writes) a JSON summary: the median counter value per dispatch of the
kernel and of the copy, the two scale factors, and traffic_bytes = the kernel's scaled fetch +
write bytes per dispatch.
"""

import argparse
import csv
import glob
import json
import os
import statistics


def counter_rows(path):
    """Rows of the counter-collection CSV under `path` (a file or a rocprofv3 output directory)."""
    files = [path] if os.path.isfile(path) else sorted(
        glob.glob(os.path.join(path, "**", "*counter_collection*.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no counter_collection CSV under {path}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def per_dispatch(rows, counter, name_part):
    """Median over dispatches of the kernel of the counter's value (summed over its instances
    within a dispatch)."""
    by = {}
    for r in rows:
        if r.get("Counter_Name") != counter or name_part not in r.get("Kernel_Name", ""):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id")
        by[key] = by.get(key, 0.0) + float(r["Counter_Value"])
    if not by:
        raise SystemExit(f"no {counter} values for kernels matching {name_part!r}")
    return statistics.median(by.values()), len(by)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--kernel", required=True, help="substring of the kernel's (mangled) name")
    ap.add_argument("--copy-kernel", default="stream_copy_kernel")
    ap.add_argument("--copy-bytes", type=int, required=True)
    ap.add_argument("--algorithmic", type=int, default=0, help="the kernel's algorithmic bytes")
    ap.add_argument("--out")
    args = ap.parse_args()
    fr, wr = counter_rows(args.fetch), counter_rows(args.write)
    kf, nd = per_dispatch(fr, "FETCH_SIZE", args.kernel)
    kw, _ = per_dispatch(wr, "WRITE_SIZE", args.kernel)
    cf, _ = per_dispatch(fr, "FETCH_SIZE", args.copy_kernel)
    cw, _ = per_dispatch(wr, "WRITE_SIZE", args.copy_kernel)
    f_scale = args.copy_bytes / (cf * 1024.0)
    w_scale = args.copy_bytes / (cw * 1024.0)
    out = {
        "kernel": args.kernel, "dispatches": nd,
        "fetch_kib": round(kf, 2), "write_kib": round(kw, 2),
        "copy_bytes": args.copy_bytes, "copy_fetch_kib": round(cf, 2), "copy_write_kib": round(cw, 2),
        "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
        "fetch_bytes": round(kf * 1024 * f_scale), "write_bytes": round(kw * 1024 * w_scale),
    }
    out["traffic_bytes"] = out["fetch_bytes"] + out["write_bytes"]
    if args.algorithmic:
        out["algorithmic_bytes"] = args.algorithmic
        out["traffic_over_algorithmic"] = round(out["traffic_bytes"] / args.algorithmic, 3)
    s = json.dumps(out)
    print(s)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(s + "\n")


if __name__ == "__main__":
    main()
