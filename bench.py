"""Benchmark: the full Julia-1-shaped forward pass (the benchmark's config 4: 22-layer ModernBERT
encoder, hidden 768, 12 heads, GeGLU 1152, plus the head and scorer; seeded synthetic weights)
on one 293-token request per step, through the drop-in C ABI (julia_cuda_run), on one MI355X.

Prints one JSON line: `value` is GPU ms per request (HIP events, embed to logits, as the
reference's engine measures it: src/engine.rs:98-105), the better of the per-step kernels and the
persistent layer kernel; it also carries
  - the fused GEMMs' TFLOP/s and fraction of f16 MFMA peak at M >= 4096 (the metric's first part),
    each beside rocprofv3's dispatch duration of the same timed run (profiles/),
  - `roofline` for the kernel instance with the largest share of the forward's GPU time, and
    `roofline_config1` for config 1's qkv GEMM (per-layer kernel timings with HIP events,
    rotating through the 22 layers' weights, src/main.rs:307-312; the rocprofv3 figure beside),
  - `cpu_baseline`: the f32 CPU oracle (oracle/liboracle.so) on the box's host cores, on a
    bounded sample of the same workload,
  - config 4's latency distribution (mean, p50, p99 over seeded request lengths 72-1024),
  - config 5: the persistent layer kernel at 448 tokens, and the batched variant (64 requests of
    config 4's lengths concatenated, ~18.8k rows) through both paths, with per-phase GPU time,
    TFLOP/s and fraction of f16 MFMA peak.

--section runs a subset (the profiled runs of profiles/ use `--section kernels,fused_gemm
--path per-step`); the persistent kernel's cooperative launches are refused under a profiler.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "julia-cuda_amd"))

import julia_hip as jh  # noqa: E402

METRIC = "fused-GEMM TFLOP/s & % f16 MFMA peak; encoder ms/request @293 tokens"
PEAK_F16 = 2.5e15   # dense f16 MFMA, MI355X
PEAK_HBM = 8.0e12   # HBM3E bytes/s
D, I, H, L, VOCAB, FF = 768, 1152, 12, 22, 50368, 1536


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def percentile(xs, p):
    """src/serve.rs:85: the value at index round((len - 1) p) of the sorted values (Rust's
    round: halves away from zero)."""
    s = sorted(xs)
    return s[int(np.floor((len(s) - 1) * p + 0.5))]


def request(rng, n, nm=6):
    ids = rng.integers(0, VOCAB, n).astype(np.uint32)
    markers = np.sort(rng.choice(n, size=min(nm, n), replace=False)).astype(np.uint32)
    return ids, markers, 0


def lengths(rng, count):
    """Config 4's request lengths: log-normal (median 260, sigma 0.5), clipped to [72, 1024];
    mean ~293."""
    return np.clip(np.round(rng.lognormal(np.log(260.0), 0.5, count)), 72, 1024).astype(int)


def gemm_bytes(m, n, k, epi):
    """Algorithmic HBM bytes of one fused GEMM: a, w and c once (c read too with a residual),
    plus the epilogue's vectors (colsum, bias, row statistics, RoPE table rows)."""
    b = 2 * (m * k + n * k) + 2 * m * (n // 2 if epi == "lngeglu" else n)
    if epi in ("resstats", "biasresstats"):
        b += 2 * m * n + 4 * 2 * m * (n // 64)
    if epi.startswith("ln"):
        b += 4 * n + 4 * 2 * m * (k // 64)
    if "rope" in epi:
        b += 4 * 64 * m
    return b


STEP_SHAPES = {  # step: (n, k, epilogue, count per forward)
    "qkv": (3 * D, D, "lnrope", L),
    "wo": (D, D, "resstats", L),
    "wi": (2 * I, D, "lngeglu", L),
    "wo_mlp": (D, I, "resstats", L),
}


def row_bytes(step, m):
    """Algorithmic HBM bytes of the row kernels on m rows: embed (ids, the m table rows, the
    output, gamma), norm_add (x, the output, its row statistics, gamma and the type embedding),
    score over every row (the rows, w, the logits)."""
    if step == "embed":
        return 4 * m + 2 * D * m + 2 * D * m + 4 * D
    if step == "norm_add":
        return 2 * D * m + 2 * D * m + 8 * m * (D // 64) + 8 * D
    return 2 * D * m + 2 * D + 4 * m


def bandwidth_kernels(eng, m):
    """embed, norm_add and score (every row) on m rows: median us over back-to-back launches,
    GB/s of algorithmic bytes and the fraction of the HBM peak; beside each, the library's plain
    copy kernel moving the same bytes (half read, half written) in the same run: the rate this
    transfer size reaches, and the kernel's fraction of it."""
    res = {}
    for step in ("embed", "norm_add", "score"):
        _, md = eng.time_step(step, m, warmup=10, batches=5, per_batch=40)
        b = row_bytes(step, m)
        half = (b // 2 + 15) // 16 * 16
        _, cp = jh.time_copy(half, warmup=10, batches=5, per_batch=40)
        res[step] = {"us": round(md, 3), "bytes": b, "GBps": round(b / (md * 1e-6) / 1e9, 1),
                     "frac_hbm": round(b / (md * 1e-6) / PEAK_HBM, 4),
                     "copy_same_bytes_us": round(cp, 3),
                     "copy_frac_hbm": round(2 * half / (cp * 1e-6) / PEAK_HBM, 4),
                     "frac_of_copy": round(cp / md, 4)}
    return res


def attention_flops(n, window):
    pairs = n * n if window == 0 else sum(min(n, i + window + 1) - max(0, i - window) for i in range(n))
    return 4 * 64 * H * pairs


def config5_batched(lens, seed=55):
    """Config 5's batched variant: the requests concatenated (positions restarting, attention
    within each), the encoder through the per-step kernels and the persistent kernel; per-phase
    GPU ms of the per-step path with TFLOP/s and fraction of f16 MFMA peak."""
    rng = np.random.default_rng(seed)
    seqs = [rng.integers(0, VOCAB, int(n)).astype(np.uint32) for n in lens]
    rows = int(sum(lens))
    eng = jh.Engine(f"synthetic:batch_rows={rows}", max_length=1024)
    res = {"requests": len(lens), "rows": rows}
    for fused in (False, True):
        eng.encode_batch(seqs, layer_fused=fused, want_x=False)
        ms = [eng.encode_batch(seqs, layer_fused=fused, want_x=False)[1] for _ in range(3)]
        res["layer_kernel_ms" if fused else "per_step_ms"] = round(float(np.median(ms)), 3)
    ph = eng.encode_batch_phases(seqs)
    eng.close()
    n_glob = sum(1 for l in range(L) if l % 3 == 0)  # every third layer global
    flops = {s: 2 * rows * n * k * L for s, (n, k, _, _) in STEP_SHAPES.items()}
    flops["attention"] = sum(n_glob * attention_flops(int(n), 0) + (L - n_glob) * attention_flops(int(n), 64)
                             for n in lens)
    phases = {}
    for s, ms in ph.items():
        tf = flops[s] / (ms * 1e-3) / 1e12
        phases[s] = {"ms": round(ms, 3), "TFLOPs": round(tf, 1), "frac_peak": round(tf * 1e12 / PEAK_F16, 4)}
    res["phases_per_step"] = phases
    gemm_fl = sum(flops[s] for s in STEP_SHAPES)
    gemm_ms = sum(ph[s] for s in STEP_SHAPES)
    res["gemm_TFLOPs"] = round(gemm_fl / (gemm_ms * 1e-3) / 1e12, 1)
    res["gemm_frac_peak"] = round(gemm_fl / (gemm_ms * 1e-3) / PEAK_F16, 4)
    return res


def config4_throughput(reqs, fused, spec, per_step_engine):
    """Multi-request throughput on config 4's requests: one by one through julia_cuda_run's
    queue, against julia_hip_run_batched's passes over concatenated rows (all requests in one
    pass, and passes of at most 4096 rows). Requests/s and tokens/s over the host's wall clock
    around the call (inputs from host memory, logits back), the summed pass GPU ms beside it,
    and the largest logit difference to the one-by-one results."""
    tokens = sum(len(r[0]) for r in reqs)
    res = {"requests": len(reqs), "tokens": tokens, "path": "layer kernel" if fused else "per step"}

    def measure(eng, batched, reps=3):
        eng.run(reqs, layer_fused=fused, batched=batched)
        best, out = None, None
        for _ in range(reps):
            t0 = time.perf_counter()
            lg, ms = eng.run(reqs, layer_fused=fused, batched=batched)
            wall = time.perf_counter() - t0
            if best is None or wall < best[0]:
                best, out = (wall, ms), lg
        wall, ms = best
        gpu = float(np.sum(np.unique(ms))) if batched else float(np.sum(ms))
        return out, {"wall_ms": round(wall * 1e3, 3), "gpu_ms": round(gpu, 3),
                     "requests_per_s": round(len(reqs) / wall, 1),
                     "tokens_per_s": round(tokens / wall, 0)}

    ref, res["one_by_one"] = measure(per_step_engine, False)
    for rows in (tokens, 4096):
        eng = jh.Engine(spec, max_length=1024, batch_rows=rows)
        lg, r = measure(eng, True)
        eng.close()
        r["max_logit_diff"] = float(np.max(np.abs(np.concatenate(lg) - np.concatenate(ref))))
        res[f"batched_{rows}_rows"] = r
    return res


SECTIONS = ("forward", "kernels", "config2", "config3", "fused_gemm", "config5", "config4", "cpu")
BIG_SPEC = "synthetic:layers=4,max_positions=20480"
# rocprofv3 dispatch durations of bench.py's own timed kernel runs (kernel_trace.py over a
# --kernel-trace run of `bench.py --section kernels,fused_gemm`), keyed by run label.
ROCPROF_FILE = os.path.join(ROOT, "profiles", "bench_kernels_rocprof.json")


def load_rocprof():
    if not os.path.exists(ROCPROF_FILE):
        return {}
    with open(ROCPROF_FILE) as fh:
        return json.load(fh).get("runs", {})


def path_ms(t):
    """(mean, median, wall) ms of one path of the forward, or None when it was not timed."""
    if not np.isfinite(t[0]):
        return None
    return {"mean": round(t[0], 4), "median": round(t[1], 4), "wall": round(t[2], 4)}


def gemm_instance(m, n, k, bm, epi, cus):
    """The kernel instance the engine launches for an m x n x k GEMM with tile height bm (one
    K split)."""
    if bm >= 128:
        return f"gemm_big<{bm}, {jh.EPI[epi]}, false>"
    if (n // 64) * -(-m // bm) <= cus and k >= 256:  # the eight-wave instance: a block a CU at most
        most = (k // 32 + 7) // 8  # K steps of the busiest wave: its K path
        path = 3 if most <= 3 else 5 if most <= 5 else 6 if most <= 6 and bm <= 32 else 1
        return f"gemm_lat1<{bm}, {jh.EPI[epi]}, {path}>"
    return f"gemm_lat<{bm}, {jh.EPI[epi]}>"


def roofline(kern, steps, kname):
    """The roofline entry of one kernel instance at 293 tokens over the steps that run it: the
    algorithmic bytes (or flops) of the forward's launches of it over their HIP-event time
    (bench.py, live), beside the same over rocprofv3's dispatch durations of the same timed runs
    (profiles/), and the HBM traffic per launch from the committed counter passes."""
    byt = sum(kern[s]["bytes"] for s in steps)
    fl = sum(kern[s]["flops"] for s in steps)
    us = sum(kern[s]["us"] for s in steps)
    rus = [kern[s].get("rocprof_us") for s in steps]
    rus = sum(rus) if all(r is not None for r in rus) else None
    shapes = ", ".join(f"{s} gemm_{STEP_SHAPES[s][2]} M=293 N={STEP_SHAPES[s][0]} K={STEP_SHAPES[s][1]}"
                       for s in steps)
    hbm = byt / PEAK_HBM >= fl / PEAK_F16
    if hbm:
        ach, peak, unit, work = byt / (us * 1e-6) / 1e9, PEAK_HBM / 1e9, "GB/s", byt
    else:
        ach, peak, unit, work = fl / (us * 1e-6) / 1e12, PEAK_F16 / 1e12, "TFLOP/s", fl
    r = {"kernel": f"{kname}: {shapes}", "bound": "hbm" if hbm else "mfma", "achieved": round(ach, 1),
         "peak": peak, "unit": unit, "frac": round(ach / peak, 4), "traffic": None,
         "algorithmic_bytes" if hbm else "algorithmic_flops": work, "us": round(us / len(steps), 3)}
    if rus is not None:
        ach_r = (work / (rus * 1e-6)) / (1e9 if hbm else 1e12)
        r["rocprof_us"] = round(rus / len(steps), 3)
        r["frac_rocprof"] = round(ach_r / peak, 4)
    # HBM bytes per launch from the committed rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE,
    # scaled by the library's copy kernel), when they are of this kernel and these shapes.
    tr = []
    for s in steps:
        tfile = os.path.join(ROOT, "profiles", f"traffic_{s}_293.json")
        if os.path.exists(tfile):
            with open(tfile) as fh:
                t = json.load(fh)
            if t.get("kernel") == kname:
                tr.append(t["traffic_bytes"])
    if len(tr) == len(steps):
        r["traffic"] = round(sum(tr) / len(steps))
        r["traffic_over_algorithmic"] = round(sum(tr) / byt, 3)
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="forward timing only")
    ap.add_argument("--path", choices=("both", "per-step", "fused"), default="both",
                    help="time only this path of the forward pass")
    ap.add_argument("--section", default="all",
                    help="comma-separated parts to run: " + ", ".join(SECTIONS) + " (all: every "
                         "one; without forward the line carries only the parts run, for profiling)")
    ap.add_argument("--trace-labels", default="",
                    help="write the ordered list of timed kernel runs (label, kernel instance, "
                         "warm-up and timed launches) to this JSON file, for kernel_trace.py")
    args = ap.parse_args()
    sections = SECTIONS if args.section == "all" else tuple(args.section.split(","))
    for sec in sections:
        if sec not in SECTIONS:
            ap.error(f"no section {sec!r}")
    if args.quick:
        sections = ("forward",)
    coop = ("forward" in sections and args.path != "per-step") or "config5" in sections or \
        ("config4" in sections and args.path != "per-step")
    if coop:
        jh.refuse_cooperative_under_profiler(
            "bench.py with the persistent kernel (the forward's fused path, config5, or config4 "
            "on it; use --path per-step and leave out config5)")
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(requests are independent: the multi-GPU design is one engine per GPU)",
              file=sys.stderr)
        sys.exit(2)

    # No torch in this process: the library's own HIP runtime (the ROCm it was built with) runs
    # everything, and the device buffers of the sweeps come from it too.
    assert jh.device_count() > 0, "bench.py needs a GPU"
    rng = np.random.default_rng(293)
    eng = jh.Engine("synthetic", max_length=1024)
    info = eng.info()
    log(f"device {eng.device()}, {info.cus} CUs; weights {info.weight_bytes_f16 / 1e6:.1f} MB f16")
    req = request(rng, 293)
    labels = []  # the timed kernel runs, in launch order (--trace-labels)

    def time_step(e, step, m, label, kernel, warmup=20, batches=10, per_batch=44):
        labels.append({"label": label, "kernel": kernel, "warmup": warmup,
                       "timed": batches * per_batch})
        return e.time_step(step, m, warmup=warmup, batches=batches, per_batch=per_batch)

    out = {"metric": METRIC}
    best_fused = False
    if "forward" in sections:
        def timed(fused):  # julia_cuda_run returns after its stream has finished
            eng.run([req] * args.warmup, layer_fused=fused)
            t0 = time.perf_counter()
            _, ms = eng.run([req] * args.steps, layer_fused=fused)
            wall = (time.perf_counter() - t0) * 1e3 / args.steps
            return float(np.mean(ms)), float(np.median(ms)), wall

        skip = (float("inf"),) * 3
        per_step = timed(False) if args.path != "fused" else skip
        fused = timed(True) if args.path != "per-step" else skip
        log(f"293 tokens: per-step kernels {per_step[0]:.3f} ms GPU ({per_step[2]:.3f} wall), "
            f"layer kernel {fused[0]:.3f} ms GPU ({fused[2]:.3f} wall) (inf: not timed)")
        best_fused = fused[0] < per_step[0]
        best = fused if best_fused else per_step
        out.update({
            "value": round(best[0], 4),
            "unit": "ms/request",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(best[2], 4),
            "higher_is_better": False,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f16",
            "data": "synthetic (seeded ModernBERT-base-shaped weights and token ids)",
            "config": {
                "workload": "config 4: full forward (embed, 22-layer encoder, 2-layer head, scorer) "
                            "of one 293-token request, 6 markers",
                "d": D, "heads": H, "inter": I, "layers": L, "head_ff": FF, "vocab": VOCAB,
                "tokens": 293, "path": "layer kernel" if best_fused else "per-step kernels",
            },
            "per_step_ms": path_ms(per_step),
            "layer_kernel_ms": path_ms(fused),
        })
    prof = load_rocprof()

    # ---- per-kernel timings at 293 tokens, rotating through the layers' weights ----
    if "kernels" in sections:
        kern = {}
        for step, (n, k, epi, cnt) in STEP_SHAPES.items():
            cfg = list(jh.gemm_choose(293, n, k, info.cus, epi))
            kname = gemm_instance(293, n, k, cfg[0], epi, info.cus)
            mn, md = time_step(eng, step, 293, f"{step}@293", kname)
            kern[step] = dict(us=round(md, 3), us_min=round(mn, 3), per_forward=cnt, kernel=kname,
                              bytes=gemm_bytes(293, n, k, epi), flops=2 * 293 * n * k, config=cfg)
        for step, window in (("attention_global", 0), ("attention", None)):
            mn, md = time_step(eng, step, 293, f"{step}@293", "attention")
            kern[step] = dict(us=round(md, 3), us_min=round(mn, 3),
                              per_forward=(8 if step == "attention_global" else L),
                              bytes=2 * 293 * 4 * D,
                              flops=attention_flops(293, 0) if window == 0 else None)
        kern["attention"]["per_forward"] = L  # mixed global / window, rotating layers
        kern["attention_global"]["per_forward"] = 0  # included in "attention"
        for key, v in kern.items():
            v["total_us"] = round(v["us"] * v["per_forward"], 2)
            if v.get("bytes"):
                v["GBps"] = round(v["bytes"] / (v["us"] * 1e-6) / 1e9, 1)
            if v.get("flops"):
                v["TFLOPs"] = round(v["flops"] / (v["us"] * 1e-6) / 1e12, 2)
            r = prof.get(f"{key}@293")
            if r and r.get("kernel") == v.get("kernel", r.get("kernel")):
                v["rocprof_us"] = r["avg_us"]
        out["kernels_293"] = kern
        out["bandwidth_kernels"] = {"293_rows": bandwidth_kernels(eng, 293)}
        # The roofline: the kernel instance with the largest share of the forward's GPU time
        # (steps that share an instance count together), and config 1's qkv GEMM beside it.
        by_inst = {}
        for step in STEP_SHAPES:
            by_inst.setdefault(kern[step]["kernel"], []).append(step)
        dom_inst = max(by_inst, key=lambda kn: sum(kern[s]["total_us"] for s in by_inst[kn]))
        out["roofline"] = roofline(kern, by_inst[dom_inst], dom_inst)
        out["roofline_config1"] = roofline(kern, ["qkv"], kern["qkv"]["kernel"])
        log("kernels at 293 tokens:", json.dumps(kern))

    # ---- config 2: the per-layer GEMM set at M=512 over tile heights x split-K ----
    # (random operands; its own scratch for the split-K partials, which the engine's chooser
    # never picks at this size)
    dev = jh.DeviceBuffer.of
    r2 = np.random.default_rng(2)
    if "config2" in sections:
        c2 = {}
        scr = jh.Scratch(1 << 24, 1 << 16)
        M2 = 512
        for step in ("wo", "wi", "wo_mlp"):
            n, k, epi, _ = STEP_SHAPES[step]
            nout = n // 2 if epi == "lngeglu" else n
            a = dev(r2.standard_normal((M2, k)).astype(np.float16))
            w = dev((r2.standard_normal(n * k) * 0.02).astype(np.float16))
            c = dev(r2.standard_normal((M2, nout)).astype(np.float16))
            st_in = dev(np.ones((M2, k // 64, 2), np.float32))
            cs = dev(np.zeros(n, np.float32))
            st_out = dev(np.zeros((M2, n // 64, 2), np.float32))
            kw = dict(stats_in=st_in.ptr, colsum=cs.ptr) if epi == "lngeglu" else \
                dict(stats_out=st_out.ptr)
            gargs = jh.gemm_args(epi, a.ptr, w.ptr, c.ptr, M2, n, k, **kw)
            grid = {}
            for bm in (32, 64, 128):
                for sp in (1, 2, 4):
                    try:
                        _, md = jh.time_gemm(gargs, bm=bm, splits=sp, scratch=scr, warmup=5,
                                             batches=5, per_batch=20)
                        grid[f"{bm}/{sp}"] = round(md, 2)
                    except jh.JuliaHipError:  # a combination the kernels do not take
                        grid[f"{bm}/{sp}"] = None
            _, md = jh.time_gemm(gargs, scratch=scr, warmup=5, batches=5, per_batch=20)
            c2[step] = {"epilogue": epi, "us_by_bm_split": grid,
                        "chosen": list(jh.gemm_choose(M2, n, k, info.cus, epi)),
                        "chosen_us": round(md, 2),
                        "TFLOPs": round(2 * M2 * n * k / (md * 1e-6) / 1e12, 1)}
            for b in (a, w, c, st_in, cs, st_out):
                b.close()
        scr.close()
        out["config2_512"] = c2
        log("config 2:", json.dumps(c2))

    # ---- config 3: attention alone, global and +-64 window ----
    if "config3" in sections:
        c3 = {}
        for n_att in (72, 293, 1024):
            q = dev(r2.standard_normal((n_att, 3 * D)).astype(np.float16))
            o = jh.DeviceBuffer(n_att * D * 2)
            for window in (0, 64):
                _, md = jh.time_attention(q.ptr, o.ptr, n_att, D, window, 1,
                                          warmup=10, batches=5, per_batch=40)
                fl = attention_flops(n_att, window)
                c3[f"n{n_att}_{'global' if window == 0 else 'window64'}"] = {
                    "us": round(md, 2), "TFLOPs": round(fl / (md * 1e-6) / 1e12, 1)}
            q.close()
            o.close()
        out["config3_attention"] = c3
        log("config 3:", json.dumps(c3))

    # ---- the fused GEMMs at M >= 4096 (the metric's TFLOP/s and % of f16 MFMA peak) ----
    if "fused_gemm" in sections:
        big = {}
        # (the full vocabulary: the embed rows of 18379 ids are mostly distinct table rows)
        eng_big = jh.Engine(BIG_SPEC, max_length=18752)
        for m in (4096, 8192, 18752):
            for step, (n, k, epi, _) in STEP_SHAPES.items():
                cfg = list(jh.gemm_choose(m, n, k, info.cus, epi))
                kname = gemm_instance(m, n, k, cfg[0], epi, info.cus)
                mn, md = time_step(eng_big, step, m, f"{step}@{m}", kname, warmup=5, batches=5,
                                   per_batch=8)
                fl = 2 * m * n * k
                big[f"{step}@{m}"] = e = dict(us=round(md, 2), TFLOPs=round(fl / (md * 1e-6) / 1e12, 1),
                                              frac_peak=round(fl / (md * 1e-6) / PEAK_F16, 4),
                                              config=cfg, kernel=kname)
                r = prof.get(f"{step}@{m}")
                if r and r.get("kernel") == kname:
                    e["rocprof_us"] = r["avg_us"]
                    e["frac_peak_rocprof"] = round(fl / (r["avg_us"] * 1e-6) / PEAK_F16, 4)
        out.setdefault("bandwidth_kernels", {})["18379_rows"] = bandwidth_kernels(eng_big, 18379)
        log("bandwidth kernels:", json.dumps(out["bandwidth_kernels"]))
        tot_fl = sum(2 * 18752 * n * k for (n, k, _, _) in STEP_SHAPES.values())
        tot_us = sum(big[f"{s}@18752"]["us"] for s in STEP_SHAPES)
        out["fused_gemm_tflops"] = round(tot_fl / (tot_us * 1e-6) / 1e12, 1)
        out["fused_gemm_frac_peak"] = round(tot_fl / (tot_us * 1e-6) / PEAK_F16, 4)
        out["fused_gemm"] = big
        log("fused GEMMs at M>=4096:", json.dumps(big))
        eng_big.close()

    # ---- config 5: the persistent layer kernel at 448 tokens, and the batched M ~ 18.8k ----
    if "config5" in sections:
        r448 = request(rng, 448)
        for fused_flag in (False, True):
            eng.run([r448] * 10, layer_fused=fused_flag)
        _, ms_s = eng.run([r448] * 50)
        _, ms_f = eng.run([r448] * 50, layer_fused=True)
        out["config5_448"] = {"per_step_ms": round(float(np.mean(ms_s)), 4),
                              "layer_kernel_ms": round(float(np.mean(ms_f)), 4)}
        out["config5_batched"] = config5_batched(lengths(np.random.default_rng(4), 64))  # config 4's requests
        log("config 5:", json.dumps(out["config5_448"]), json.dumps(out["config5_batched"]))

    # ---- config 4's latency distribution ----
    if "config4" in sections:
        lens = lengths(np.random.default_rng(4), 64)
        reqs = [request(rng, int(nn)) for nn in lens]
        path_fused = best_fused
        eng.run(reqs[:8], layer_fused=path_fused)
        _, ms = eng.run(reqs, layer_fused=path_fused)
        ms = [float(x) for x in ms]
        out["config4_lengths"] = {"requests": len(lens), "mean_tokens": round(float(lens.mean()), 1),
                                  "mean_ms": round(float(np.mean(ms)), 4),
                                  "p50_ms": round(percentile(ms, 0.5), 4),
                                  "p99_ms": round(percentile(ms, 0.99), 4)}
        out["config4_throughput"] = config4_throughput(reqs, path_fused, "synthetic", eng)
        log("config 4 throughput:", json.dumps(out["config4_throughput"]))
    eng.close()
    if args.trace_labels:
        with open(args.trace_labels, "w") as fh:
            json.dump(labels, fh, indent=1)

    # ---- the CPU baseline: the f32 oracle on the host cores, a bounded sample ----
    if "cpu" in sections and not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O

        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        nproc = len(os.sched_getaffinity(0))
        model = O.Model(O.cfg())
        ids, markers, q = req
        model.forward(ids, q, markers)  # warm-up
        times = []
        t_end = time.perf_counter() + 15.0
        while time.perf_counter() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            model.forward(ids, q, markers)
            times.append((time.perf_counter() - t0) * 1e3)
        out["cpu_baseline"] = {"value": round(float(np.median(times)), 2), "unit": "ms/request",
                               "cores": threads, "nproc": nproc, "kind": "port",
                               "sample": f"{len(times)} forward passes of the same 293-token "
                                         "request (22-layer encoder + head, f32, LayerNorms in "
                                         f"f64), median, OpenMP over {threads} threads "
                                         f"(OMP_NUM_THREADS) of {nproc} host CPUs this process "
                                         "may run on; weight generation excluded"}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
