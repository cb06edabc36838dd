"""Per-kernel parity on the GPU, through the C ABI (julia_hip_gemm / _attention / _embed /
_norm_add / _score), against the CPU oracle on the same seeded inputs: the f32 reference over
unfolded weights (LayerNorms in f64) and the f16 emulation of each kernel's arithmetic.

The configurations are the benchmark's: config 1 (the fused qkv GEMM `gemm_lnrope`, M=293,
K=768, N=2304, RoPE theta 160000), config 2 (wo / wi / wo_mlp at M=512, every tile height and
split-K), config 3 (attention, 12 heads x 64, n in {72, 293, 1024}, global and +-64 window),
plus the head's four epilogues, the bandwidth kernels, and MFMA-bound shapes (M >= 4096)."""

import numpy as np
import pytest

import julia_hip as jh
import oracle as O
from checks import (ATTN_REL, EMU_REL, GEMM_REL, check_stats, compare, f32, rand16)
from conftest import f16_bits, to_dev

pytestmark = pytest.mark.gpu

EPS = 1e-5


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def scratch(torch_cuda):
    s = jh.Scratch(ws_floats=1 << 24, counters=1 << 16)
    yield s
    s.close()


def _erf_gelu(x):
    import torch

    return torch.nn.functional.gelu(torch.from_numpy(np.asarray(x, np.float64))).numpy()


def gemm_problem(kind, m, n, k, seed=1, theta=160000.0):
    """Inputs (f16 bits / f32 arrays), the f32 reference output and the emulation's."""
    rng = np.random.default_rng(seed)
    epi = jh.EPI[kind]
    P = dict(kind=kind, epi=epi, m=m, n=n, k=k)
    if kind in ("rope", "lnrope", "lngeglu", "lnbias", "lnbiasrelu", "lnbiasgelu"):
        x16 = rand16(rng, (m, k), std=1.0, mean=0.1)
        W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        x = f32(x16)
        P["a"] = x16
        if kind == "rope":
            w16 = O.to_f16_bits(W)
            ref = O.linear(x, W)
        elif kind in ("lnrope", "lngeglu"):
            w16, cs = O.fold_layernorm(W, gamma)
            ref = O.linear(O.layernorm_rows(x, gamma, None, EPS), W)
            P["stats_in"], P["colsum"] = O.row_stats(x16), cs
        else:
            beta = (0.05 * rng.standard_normal(k)).astype(np.float32)
            b = (0.02 * rng.standard_normal(n)).astype(np.float32)
            w16, cs, bias = O.fold_layernorm_bias(W, gamma, beta, b)
            ref = O.linear(O.layernorm_rows(x, gamma, beta, EPS), W, b)
            P["stats_in"], P["colsum"], P["bias"] = O.row_stats(x16), cs, bias
            if kind == "lnbiasrelu":
                ref = np.maximum(ref, 0)
            if kind == "lnbiasgelu":
                ref = _erf_gelu(ref)
        if kind in ("rope", "lnrope"):
            table = O.rope_table(theta, m)
            ref = O.rope_apply(ref, table)
            P["rope"] = table
        if kind == "lngeglu":
            rows = O.geglu_rows(n // 2)
            w16 = np.ascontiguousarray(w16[rows])
            P["colsum"] = np.ascontiguousarray(P["colsum"][rows])
            ref = O.geglu(ref)
        P["w"] = w16
    else:  # resstats, biasresstats: c = res + a . W^T (+ b)
        a16 = rand16(rng, (m, k))
        W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        w16 = O.to_f16_bits(W)
        res16 = rand16(rng, (m, n))
        ref = f32(res16) + O.linear(f32(a16), W)
        if kind == "biasresstats":
            b = (0.02 * rng.standard_normal(n)).astype(np.float32)
            ref = ref + b
            P["bias"] = b
        P.update(a=a16, w=w16, res=res16)
    P["ref"] = ref
    emu = O.emu_gemm(P["a"], P["w"], epi, stats_in=P.get("stats_in"), colsum=P.get("colsum"),
                     eps=EPS, bias=P.get("bias"), rope=P.get("rope"),
                     rope_cols=(2 * (n // 3)) if "rope" in kind else 0, c16=P.get("res"))
    if isinstance(emu, tuple):
        P["emu"], P["emu_stats"] = emu
    else:
        P["emu"] = emu
    return P


def run_gemm(torch, P, bm, splits, scratch):
    m, n, k = P["m"], P["n"], P["k"]
    dev = {key: to_dev(torch, P[key]) for key in ("a", "stats_in", "colsum", "bias", "rope")
           if key in P}
    dev["w"] = to_dev(torch, O.pack_frag(P["w"]))  # the kernels take w in fragment order
    ncols = n // 2 if P["kind"] == "lngeglu" else n
    c = to_dev(torch, P["res"]) if "res" in P else torch.zeros((m, ncols), dtype=torch.float16,
                                                               device="cuda")
    st = torch.zeros((m, n // 64, 2), dtype=torch.float32, device="cuda") if "res" in P else None
    args = jh.gemm_args(P["epi"], dev["a"].data_ptr(), dev["w"].data_ptr(), c.data_ptr(), m, n, k,
                        stats_in=dev["stats_in"].data_ptr() if "stats_in" in dev else 0,
                        colsum=dev["colsum"].data_ptr() if "colsum" in dev else 0, eps=EPS,
                        bias=dev["bias"].data_ptr() if "bias" in dev else 0,
                        rope=dev["rope"].data_ptr() if "rope" in dev else 0,
                        rope_rows=m, stats_out=st.data_ptr() if st is not None else 0)
    jh.gemm(args, bm=bm, splits=splits, scratch=scratch,
            stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return f16_bits(c), (st.cpu().numpy() if st is not None else None)


def check_gemm(P, out16, stats, label):
    rel, mrel = compare(f32(out16), P["ref"], GEMM_REL, what=f"{label} vs f32")
    erel, _ = compare(f32(out16), f32(P["emu"]), EMU_REL, what=f"{label} vs emulation")
    if stats is not None:
        check_stats(out16, stats, what=f"{label} stats")
    say(f"  {label}: vs f32 {rel:.2e} (max {mrel:.2e}), vs emulation {erel:.2e}")


# ---- config 1: the fused qkv GEMM -------------------------------------------------------
@pytest.mark.parametrize("bm,splits", [(0, 1), (16, 1), (32, 1), (64, 1), (32, 2), (16, 3),
                                       (128, 1), (256, 1), (128, 2), (256, 4)])
def test_config1_gemm_lnrope(torch_cuda, scratch, bm, splits):
    say(f"config 1 gemm_lnrope M=293 K=768 N=2304 bm={bm} splits={splits}")
    P = gemm_problem("lnrope", 293, 2304, 768, seed=11)
    out, _ = run_gemm(torch_cuda, P, bm, splits, scratch)
    check_gemm(P, out, None, f"lnrope bm={bm} z={splits}")


def test_gemm_rope_layer0(torch_cuda, scratch):
    say("gemm_rope (layer 0, no LayerNorm) M=72 N=2304 K=768, theta 10000")
    P = gemm_problem("rope", 72, 2304, 768, seed=12, theta=10000.0)
    out, _ = run_gemm(torch_cuda, P, 0, 1, scratch)
    check_gemm(P, out, None, "rope")


# ---- config 2: the per-layer GEMM set at M=512, every tile height and split-K -------------
CONFIG2 = [("resstats", 768, 768), ("lngeglu", 2304, 768), ("resstats", 768, 1152)]


@pytest.mark.parametrize("kind,n,k", CONFIG2, ids=["wo", "wi", "wo_mlp"])
@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("splits", [1, 2, 4])
def test_config2_layer_gemms(torch_cuda, scratch, kind, n, k, bm, splits):
    say(f"config 2 {kind} M=512 N={n} K={k} bm={bm} splits={splits}")
    P = gemm_problem(kind, 512, n, k, seed=21 + n + k)
    out, st = run_gemm(torch_cuda, P, bm, splits, scratch)
    check_gemm(P, out, st, f"{kind} n={n} k={k} bm={bm} z={splits}")


# ---- the head's epilogues -----------------------------------------------------------------
@pytest.mark.parametrize("kind,n,k", [("lnbias", 2304, 768), ("biasresstats", 768, 768),
                                      ("lnbiasrelu", 1536, 768), ("biasresstats", 768, 1536),
                                      ("lnbiasgelu", 768, 768)])
def test_head_gemms(torch_cuda, scratch, kind, n, k):
    say(f"head {kind} M=293 N={n} K={k}")
    P = gemm_problem(kind, 293, n, k, seed=31 + n)
    out, st = run_gemm(torch_cuda, P, 0, 1, scratch)
    check_gemm(P, out, st, f"{kind} n={n} k={k}")


# ---- the eight-wave latency kernel's K paths ----------------------------------------------
# gemm_lat1 (grids of at most a block a CU) fixes its waves' K path per instance from K: wave w
# of 8 takes K units [w U / 8, (w + 1) U / 8) of U = K / 32, all in one chunk when the busiest
# wave has at most three (K <= 768), five (K <= 1280) or, on tiles of up to 32 rows, six
# (K <= 1536) units, with a's lines staged through the wave's LDS slot, else in the chunked
# loop. K at and around each boundary (320, 832 and 1344: waves whose range starts in the middle
# of a 128-byte line; 1344 and 1536 on 48 and 64 rows, and 3072: the loop), every tile height,
# M = 293 (rows past m in the last tile). Grids: 12 or 36 column tiles x 5-19 row tiles,
# at most 252 blocks, so the eight-wave kernel runs on a 256-CU MI355X.
LAT1_KS = [256, 320, 768, 832, 1152, 1280, 1344, 1536, 3072]


@pytest.mark.parametrize("k", LAT1_KS)
@pytest.mark.parametrize("kind,n,bm", [("resstats", 768, 16), ("resstats", 768, 32),
                                       ("lngeglu", 2304, 48), ("lnrope", 2304, 48),
                                       ("resstats", 768, 64)])
def test_eight_wave_latency_tile_k_paths(torch_cuda, scratch, kind, n, bm, k):
    say(f"eight-wave latency tile {kind} M=293 N={n} K={k} bm={bm}")
    P = gemm_problem(kind, 293, n, k, seed=71 + k + bm)
    out, st = run_gemm(torch_cuda, P, bm, 1, scratch)
    check_gemm(P, out, st, f"{kind} n={n} k={k} bm={bm}")


# ---- MFMA-bound sizes ---------------------------------------------------------------------
# Every epilogue on the throughput tiles (128 x 128 and 256 x 256), M not a multiple of either.
BIG_EPIS = [("lnrope", 2304, 768), ("rope", 2304, 768), ("lngeglu", 2304, 768),
            ("resstats", 768, 768), ("resstats", 768, 1152), ("lnbias", 2304, 768),
            ("biasresstats", 768, 1536), ("lnbiasrelu", 1536, 768), ("lnbiasgelu", 768, 768)]


@pytest.mark.parametrize("kind,n,k", BIG_EPIS, ids=[f"{a}-{b}-{c}" for a, b, c in BIG_EPIS])
@pytest.mark.parametrize("bm", [128, 192, 256])
def test_big_tiles_every_epilogue(torch_cuda, scratch, kind, n, k, bm):
    say(f"big tiles {kind} M=2100 N={n} K={k} bm={bm}")
    P = gemm_problem(kind, 2100, n, k, seed=51 + n + k)
    out, st = run_gemm(torch_cuda, P, bm, 1, scratch)
    check_gemm(P, out, st, f"{kind} M=2100 n={n} k={k} bm={bm}")


@pytest.mark.parametrize("kind,n,k", [("lnrope", 2304, 768), ("resstats", 768, 1152),
                                      ("lngeglu", 2304, 768), ("lnbiasgelu", 768, 768)])
def test_chooser_at_row_edges(torch_cuda, scratch, kind, n, k):
    """The chooser's own pick (bm = 0) at row counts around the tile heights (1, 16, 48, 256)
    and the switch from the one-block-a-CU latency kernel to the two-a-CU one and to the
    throughput tiles, against the f32 reference and the emulation."""
    for m in (1, 15, 17, 47, 49, 255, 257, 1023, 2049):
        P = gemm_problem(kind, m, n, k, seed=500 + m + n)
        out, st = run_gemm(torch_cuda, P, 0, 1, scratch)
        check_gemm(P, out, st, f"{kind} m={m} chosen {tuple(jh.gemm_choose(m, n, k, 256, P['epi']))}")


# K split on the throughput tiles: the last arriver's sum in split order, then every kind of
# epilogue (RoPE, GeGLU, residual + statistics, bias + residual), rows past m in the last band.
SPLIT_EPIS = [("lnrope", 2304, 768), ("lngeglu", 2304, 768), ("resstats", 768, 1152),
              ("biasresstats", 768, 1536)]


@pytest.mark.parametrize("kind,n,k", SPLIT_EPIS, ids=[f"{a}-{b}-{c}" for a, b, c in SPLIT_EPIS])
@pytest.mark.parametrize("bm,splits", [(128, 3), (192, 2), (256, 3)])
def test_big_tiles_split_k(torch_cuda, scratch, kind, n, k, bm, splits):
    say(f"big tiles split-K {kind} M=2100 N={n} K={k} bm={bm} splits={splits}")
    P = gemm_problem(kind, 2100, n, k, seed=61 + n + k)
    out, st = run_gemm(torch_cuda, P, bm, splits, scratch)
    check_gemm(P, out, st, f"{kind} M=2100 n={n} k={k} bm={bm} z={splits}")
    out1, st1 = run_gemm(torch_cuda, P, bm, splits, scratch)  # again: the counters were reset
    assert np.array_equal(out, out1), "split-K result differs between two calls"


@pytest.mark.parametrize("bm", [128, 256])
def test_large_m_lngeglu(torch_cuda, scratch, bm):
    say(f"lngeglu M=4096 N=2304 K=768 bm={bm}")
    P = gemm_problem("lngeglu", 4096, 2304, 768, seed=41)
    out, _ = run_gemm(torch_cuda, P, bm, 1, scratch)
    check_gemm(P, out, None, f"lngeglu M=4096 bm={bm}")


# ---- config 3: attention ----------------------------------------------------------------
@pytest.mark.parametrize("n", [72, 293, 1024])
@pytest.mark.parametrize("window", [0, 64])
@pytest.mark.parametrize("chunks", [1, 3])
def test_config3_attention(torch_cuda, scratch, n, window, chunks):
    say(f"config 3 attention n={n} window={window} chunks={chunks}")
    torch = torch_cuda
    rng = np.random.default_rng(100 + n + window)
    qkv16 = rand16(rng, (n, 3 * 768))
    ref = O.attention(f32(qkv16), window)
    emu = O.emu_attention(qkv16, window)
    q = to_dev(torch, qkv16)
    o = torch.zeros((n, 768), dtype=torch.float16, device="cuda")
    jh.attention(q.data_ptr(), o.data_ptr(), n, 768, window, chunks, scratch,
                 stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = f16_bits(o)
    rel, mrel = compare(f32(out), ref, ATTN_REL, what="attention vs f64")
    erel, _ = compare(f32(out), f32(emu), 2e-3, what="attention vs emulation")
    say(f"  vs f64 {rel:.2e} (max {mrel:.2e}), vs emulation {erel:.2e}")


@pytest.mark.parametrize("lens", [[300, 1024, 17, 700, 1, 513], [70, 130, 45, 200, 64], [70, 130, 45, 64]])
@pytest.mark.parametrize("window", [0, 64])
def test_attention_over_concatenated_sequences(torch_cuda, scratch, lens, window):
    """Config 5's batched attention: sequences concatenated into one set of rows, each query
    seeing only its own sequence's keys (past 2048 rows the streaming 64-query tile; 509 rows the
    slice tile or, global, 2 x 4 streaming waves; 309 rows four single-wave key groups), against
    the f64 attention of each sequence alone."""
    say(f"attention over {len(lens)} sequences ({sum(lens)} rows) window={window}")
    torch = torch_cuda
    n = sum(lens)
    rng = np.random.default_rng(300 + n + window)
    qkv16 = rand16(rng, (n, 3 * 768))
    starts = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    seg = np.zeros((n, 2), np.int32)
    for a, b in zip(starts[:-1], starts[1:]):
        seg[a:b, 0], seg[a:b, 1] = a, b
    q, sg = to_dev(torch, qkv16), to_dev(torch, seg)
    o = torch.full((n, 768), float("nan"), dtype=torch.float16, device="cuda")
    jh.attention_seg(q.data_ptr(), o.data_ptr(), n, 768, window, sg.data_ptr(), scratch,
                     stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = f32(f16_bits(o))
    for a, b in zip(starts[:-1], starts[1:]):
        ref = O.attention(f32(qkv16[a:b]), window)
        compare(out[a:b], ref, ATTN_REL, what=f"rows {a}:{b} window {window}")


def test_attention_d384_and_tail(torch_cuda, scratch):
    """The real Julia-1 width (6 heads) and a length that is not a multiple of 64 (2048 rows:
    the streaming tile with four key groups); 672 / 673 rows are the two sides of the largest
    grid of single-wave key groups that fits 256 CUs at this width."""
    torch = torch_cuda
    for n, window in [(363, 64), (363, 0), (450, 0), (1, 0), (65, 64), (2048, 0), (672, 0),
                      (673, 0), (672, 64), (673, 64)]:
        say(f"attention d=384 n={n} window={window}")
        rng = np.random.default_rng(7 + n)
        qkv16 = rand16(rng, (n, 3 * 384))
        ref = O.attention(f32(qkv16), window)
        q = to_dev(torch, qkv16)
        o = torch.zeros((n, 384), dtype=torch.float16, device="cuda")
        jh.attention(q.data_ptr(), o.data_ptr(), n, 384, window, 0, scratch,
                     stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        compare(f32(f16_bits(o)), ref, ATTN_REL, what=f"attention d=384 n={n} w={window}")


@pytest.mark.parametrize("window", [0, 64])
def test_attention_at_the_routing_edges(torch_cuda, scratch, window):
    """One sequence at d=768 on both sides of every size where attention_launch changes tile
    (global: the slice tile up to 128 rows, the streaming tile with four single-wave key groups
    up to 336 rows, then 2 x 4 waves up to 682 rows, 4 x 4 up to 1365, 4 x 2 up to 2730, 4 x 1
    past it; window: the slice tile up to 97 rows, four single-wave key groups up to 336, the
    slice tile up to 768 rows, then the streaming tile), and at lengths around the 16-, 32- and
    64-row block edges, against the f64 attention."""
    torch = torch_cuda
    for n in (2, 17, 63, 64, 65, 97, 98, 128, 129, 292, 293, 336, 337, 400, 682, 683, 768, 769,
              1365, 1366, 2730, 2731):
        rng = np.random.default_rng(900 + n + window)
        qkv16 = rand16(rng, (n, 3 * 768))
        ref = O.attention(f32(qkv16), window)
        q = to_dev(torch, qkv16)
        o = torch.full((n, 768), float("nan"), dtype=torch.float16, device="cuda")
        jh.attention(q.data_ptr(), o.data_ptr(), n, 768, window, 1, scratch,
                     stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rel, mrel = compare(f32(f16_bits(o)), ref, ATTN_REL, what=f"attention n={n} window={window}")
        say(f"  n={n} window={window}: vs f64 {rel:.2e} (max {mrel:.2e})")


# ---- the bandwidth kernels ----------------------------------------------------------------
@pytest.mark.parametrize("d", [384, 768])
def test_embed(torch_cuda, d):
    say(f"embed d={d}")
    torch = torch_cuda
    rng = np.random.default_rng(5)
    vocab, n = 1000, 293
    table16 = rand16(rng, (vocab, d))
    gamma = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ids = rng.integers(0, vocab, n).astype(np.uint32)
    emu = O.emu_embed(table16, gamma, ids, EPS)
    ref = O.layernorm_rows(f32(table16)[ids], gamma, None, EPS)
    t, g, i = to_dev(torch, table16), to_dev(torch, gamma), to_dev(torch, ids.view(np.int32))
    x = torch.zeros((n, d), dtype=torch.float16, device="cuda")
    jh.embed(i.data_ptr(), n, t.data_ptr(), vocab, d, g.data_ptr(), EPS, x.data_ptr(),
             stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = f16_bits(x)
    u = O.ulps(out, emu)
    assert u.max() <= 1, f"embed is {u.max()} ulp off the emulation"
    compare(f32(out), ref, 2e-3, what="embed vs f64 LayerNorm")


@pytest.mark.parametrize("d", [384, 768])
def test_norm_add(torch_cuda, d):
    say(f"norm_add d={d}")
    torch = torch_cuda
    rng = np.random.default_rng(6)
    n = 293
    x16 = rand16(rng, (n, d), std=3.0, mean=0.5)
    gamma = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    add = (0.1 * rng.standard_normal(d)).astype(np.float32)
    emu, _ = O.emu_norm_add(x16, gamma, add, EPS)
    x, g, a = to_dev(torch, x16), to_dev(torch, gamma), to_dev(torch, add)
    out = torch.zeros((n, d), dtype=torch.float16, device="cuda")
    st = torch.zeros((n, d // 64, 2), dtype=torch.float32, device="cuda")
    jh.norm_add(x.data_ptr(), n, d, g.data_ptr(), a.data_ptr(), EPS, out.data_ptr(), st.data_ptr(),
                stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    o16 = f16_bits(out)
    # LN(x) . gamma + add cancels to small values in places, where the f32 summation order of
    # the mean and variance moves a value by more than one of its (tiny) f16 steps.
    u = O.ulps(o16, emu)
    assert u.max() <= 4 and (u > 1).mean() < 1e-3, f"norm_add: {u.max()} ulp off the emulation"
    compare(f32(o16), f32(emu), EMU_REL, what="norm_add vs emulation")
    check_stats(o16, st.cpu().numpy(), "norm_add stats")
    ref = O.layernorm_rows(f32(x16), gamma, None, EPS) + add
    compare(f32(o16), ref, 2e-3, what="norm_add vs f64")


def test_score(torch_cuda):
    say("score")
    torch = torch_cuda
    rng = np.random.default_rng(8)
    n, d = 293, 768
    y16 = rand16(rng, (n, d))
    w16 = rand16(rng, (d,), std=0.02)
    markers = np.array([0, 5, 100, 292, 17], np.uint32)
    ref = f32(y16)[markers].astype(np.float64) @ f32(w16).astype(np.float64) + 0.25
    y, w, mk = to_dev(torch, y16), to_dev(torch, w16), to_dev(torch, markers.view(np.int32))
    lg = torch.zeros(len(markers), dtype=torch.float32, device="cuda")
    jh.score(y.data_ptr(), n, d, w.data_ptr(), 0.25, mk.data_ptr(), len(markers), lg.data_ptr(),
             stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_allclose(lg.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


def test_gemm_rejects_bad_shapes(torch_cuda, scratch):
    """gemm::launch's preconditions (src/gemm.rs:262-329) are errors, not launches."""
    torch = torch_cuda
    a = torch.zeros((64, 96), dtype=torch.float16, device="cuda")
    w = torch.zeros((64, 96), dtype=torch.float16, device="cuda")
    c = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    args = jh.gemm_args("resstats", a.data_ptr(), w.data_ptr(), c.data_ptr(), 64, 64, 96,
                        stats_out=c.data_ptr())
    with pytest.raises(jh.JuliaHipError, match="multiple of 64"):
        jh.gemm(args, 32, 1, scratch)
    args = jh.gemm_args("resstats", a.data_ptr(), w.data_ptr(), c.data_ptr(), 64, 64, 64,
                        stats_out=c.data_ptr())
    with pytest.raises(jh.JuliaHipError, match="leave a wave no K step"):
        jh.gemm(args, 32, 1, scratch)  # k = 64: two K steps for four waves
    args = jh.gemm_args("lnrope", a.data_ptr(), w.data_ptr(), c.data_ptr(), 64, 64, 64)
    with pytest.raises(jh.JuliaHipError, match="LayerNorm inputs"):
        jh.gemm(args, 32, 1, scratch)
