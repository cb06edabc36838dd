"""The persistent layer kernel's per-phase profile from its own timestamps (the reference's
src/profile.rs:84-241 over kernels/src/prof.rs's stamps).

    python julia-cuda_amd/profile.py [--tokens 293] [--layer 1 | -1] [--spec synthetic]

Per phase: the span (first block's start to last block's end), the mean busy time per block
(its start to its end stamp), the hand-over (the last end of this phase to the first start of
the next: the barrier), and the CUs used. Times in microseconds (the stamps' clock is 100 MHz).
"""

import argparse
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import julia_hip as jh  # noqa: E402

PHASES = ["qkv", "attention", "wo", "wi", "wo_mlp"]
TICK_US = 0.01  # 100 MHz


def summarize(stamps):
    """stamps: [blocks][PROF_WORDS] u64 (one layer). Returns a list of per-phase dicts; a GEMM
    phase also gets its first tasks' stage times (inputs, mfma, reduce, epilogue: the mean over
    blocks of each stage's duration, the first from the phase's start)."""
    s = stamps.astype(np.int64)
    t0 = s[:, 0].min()
    rows = []
    for p, name in enumerate(PHASES):
        st, en = s[:, 2 * p], s[:, 2 * p + 1]
        ok = (st > 0) & (en > 0)
        if not ok.any():
            continue
        st, en = st[ok], en[ok]
        row = {"phase": name, "start_us": (st.min() - t0) * TICK_US,
               "span_us": (en.max() - st.min()) * TICK_US,
               "busy_us": float(np.mean(en - st)) * TICK_US,
               "max_busy_us": float(np.max(en - st)) * TICK_US,
               "cus": int(len(np.unique(s[ok, 10])))}
        if p + 1 < len(PHASES):
            nst = s[:, 2 * p + 2]
            nst = nst[nst > 0]
            if len(nst):
                row["handover_us"] = (nst.min() - en.max()) * TICK_US
                row["barrier_wait_us"] = float(np.mean(nst - s[ok, 2 * p + 1][: len(nst)])) * TICK_US
        if name == "attention":
            sub = s[:, 12:15]
            okb = ok & (sub > 0).all(axis=1)
            if okb.any():
                d = np.diff(np.concatenate([s[okb, 2 * p][:, None], sub[okb]], axis=1), axis=1)
                for k, name_ in enumerate(("inputs_us", "compute_us", "store_us")):
                    row[name_] = float(np.mean(d[:, k])) * TICK_US
                    row["max_" + name_] = float(np.max(d[:, k])) * TICK_US
        g = {"qkv": 0, "wo": 1, "wi": 2, "wo_mlp": 3}.get(name)
        if g is not None:
            sub = s[:, 16 + 4 * g: 20 + 4 * g]
            okb = ok & (sub > 0).all(axis=1)
            if okb.any():
                d = np.diff(np.concatenate([s[okb, 2 * p][:, None], sub[okb]], axis=1), axis=1)
                for k, name_ in enumerate(("inputs_us", "mfma_us", "reduce_us", "epilogue_us")):
                    row[name_] = float(np.mean(d[:, k])) * TICK_US
        rows.append(row)
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=293)
    ap.add_argument("--layer", type=int, default=1, help="-1: the whole encoder, one launch")
    ap.add_argument("--spec", default="synthetic")
    args = ap.parse_args()
    jh.refuse_cooperative_under_profiler("profile.py (the persistent kernel's stamps)")
    e = jh.Engine(args.spec, max_length=max(1024, args.tokens))
    e.profile_layer(args.tokens, args.layer)  # warm-up
    plan, stamps = e.profile_layer(args.tokens, args.layer)
    print(f"layer {args.layer}, {args.tokens} tokens, {stamps.shape[0]} blocks, plan "
          f"bm {list(plan[:4])} splits {list(plan[4:8])} kv {list(plan[8:])}")
    if args.layer >= 0:
        for r in summarize(stamps[:, 0]):
            print("  " + ", ".join(f"{k} {v:.2f}" if isinstance(v, float) else f"{k} {v}"
                                   for k, v in r.items()))
        return
    s = stamps.astype(np.int64)
    t0 = s[:, 0, 0][s[:, 0, 0] > 0].min()
    end = s[:, -1, 9][s[:, -1, 9] > 0].max()
    print(f"  encoder span {(end - t0) * TICK_US:.2f} us over {s.shape[1]} layers")
    per = {}
    for li in range(s.shape[1]):
        for r in summarize(stamps[:, li]):
            per.setdefault(r["phase"], []).append(r)
    for name, rows in per.items():
        keys = [k for k in rows[0] if k not in ("phase", "start_us", "cus")]
        print(f"  {name}: " + ", ".join(f"{k} {np.mean([r[k] for r in rows if k in r]):.2f}"
                                         for k in keys))


if __name__ == "__main__":
    main()
