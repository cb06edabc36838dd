"""The persistent layer kernel's per-phase profile from its own timestamps (the reference's
src/profile.rs:84-241 over kernels/src/prof.rs's stamps).

    python julia-cuda_amd/profile.py [--tokens 293] [--layer 1] [--spec synthetic]

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
    """stamps: [blocks][16] u64. Returns a list of per-phase dicts."""
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
        rows.append(row)
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=293)
    ap.add_argument("--layer", type=int, default=1)
    ap.add_argument("--spec", default="synthetic")
    args = ap.parse_args()
    e = jh.Engine(args.spec, max_length=max(1024, args.tokens))
    e.profile_layer(args.tokens, args.layer)  # warm-up
    plan, stamps = e.profile_layer(args.tokens, args.layer)
    print(f"layer {args.layer}, {args.tokens} tokens, {len(stamps)} blocks, plan "
          f"bm {list(plan[:4])} splits {list(plan[4:8])} kv {list(plan[8:])}")
    for r in summarize(stamps):
        print("  " + ", ".join(f"{k} {v:.2f}" if isinstance(v, float) else f"{k} {v}"
                               for k, v in r.items()))


if __name__ == "__main__":
    main()
