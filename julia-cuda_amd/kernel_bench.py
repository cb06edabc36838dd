"""Runs one encoder step of the engine repeatedly, for profilers (rocprofv3 --kernel-trace /
--pmc): the same launches as the forward pass, rotating through the layers' weights, plus a
plain device-to-device copy of a known size to calibrate byte counters against.

    python julia-cuda_amd/kernel_bench.py --step wi --tokens 293 --iters 200 --copy-mb 64
    python julia-cuda_amd/kernel_bench.py --step embed,norm_add,score --tokens 18379 \
        --spec synthetic:layers=2,max_positions=20480
    python julia-cuda_amd/kernel_bench.py --batch 64 --iters 3 --copy-mb 0
    python julia-cuda_amd/kernel_bench.py --requests 64 --iters 3

Prints the step's median time per call (HIP events) and the copy's bytes. With --batch N: config
5's batched encoder instead (N requests of config 4's seeded lengths concatenated, per-step
kernels then the persistent kernel, --iters times each; refused under a profiler, since the
persistent kernel is a cooperative launch). With --requests N: N such requests
(6 markers each, question types in turn) through julia_hip_run_batched as one pass, the whole
forward pass (embed, encoder, head, scorer), --iters times.
"""

import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import julia_hip as jh  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--step", default="qkv",
                    help="one of " + ", ".join(jh.Engine.STEPS) + ", or several, comma-separated")
    ap.add_argument("--tokens", type=int, default=293)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--bm", type=int, default=0)
    ap.add_argument("--splits", type=int, default=1)
    ap.add_argument("--copy-mb", type=int, default=64)
    ap.add_argument("--spec", default="synthetic")
    ap.add_argument("--batch", type=int, default=0)
    ap.add_argument("--requests", type=int, default=0)
    args = ap.parse_args()
    if args.requests:
        import numpy as np
        rng = np.random.default_rng(4)
        lens = np.clip(np.round(rng.lognormal(np.log(260.0), 0.5, args.requests)), 72, 1024).astype(int)
        reqs = []
        for i, n in enumerate(lens):
            ids = rng.integers(0, 50368, int(n)).astype(np.uint32)
            reqs.append((ids, np.sort(rng.choice(int(n), 6, replace=False)).astype(np.uint32), i % 3))
        e = jh.Engine("synthetic", max_length=1024, batch_rows=int(lens.sum()))
        for _ in range(args.iters):
            _, ms = e.run(reqs, batched=True)
            print(f"{args.requests} requests ({int(lens.sum())} rows) in one pass: {ms[0]:.3f} ms",
                  flush=True)
        e.close()
        return
    if args.batch:
        jh.refuse_cooperative_under_profiler("--batch (its persistent-kernel pass)")
        import numpy as np
        rng = np.random.default_rng(4)
        lens = np.clip(np.round(rng.lognormal(np.log(260.0), 0.5, args.batch)), 72, 1024).astype(int)
        seqs = [rng.integers(0, 50368, int(n)).astype(np.uint32) for n in lens]
        e = jh.Engine(f"synthetic:batch_rows={int(lens.sum())}", max_length=1024)
        for fused in (False, True):
            ms = [e.encode_batch(seqs, layer_fused=fused, want_x=False)[1] for _ in range(args.iters)]
            print(f"batch of {args.batch} ({int(lens.sum())} rows), {'persistent' if fused else 'per-step'}: "
                  f"{sorted(ms)[len(ms) // 2]:.3f} ms", flush=True)
        e.close()
        return
    steps = args.step.split(",")
    for st in steps:
        if st not in jh.Engine.STEPS:
            ap.error(f"no step {st!r}")
    e = jh.Engine(args.spec, max_length=max(1024, args.tokens))
    for st in steps:
        mn, md = e.time_step(st, args.tokens, args.bm, args.splits, warmup=10, batches=1,
                             per_batch=args.iters)
        print(f"{st} at {args.tokens} tokens: {md:.2f} us per call", flush=True)
    if args.copy_mb:
        nbytes = args.copy_mb << 20
        mn, md = jh.time_copy(nbytes, warmup=2, batches=1, per_batch=5)
        print(f"stream_copy_kernel: {nbytes} bytes read and {nbytes} written per call, "
              f"{md:.2f} us, {2 * nbytes / md / 1e3:.0f} GB/s", flush=True)
    e.close()


if __name__ == "__main__":
    main()
