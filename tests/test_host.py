"""CPU tests of the product library: it loads without a GPU and exports every symbol
include/julia_hip.h declares; its host-side logic (the synthetic generator, the weight
preparation of src/prep.rs, the tile choosers) against the oracle's independent restatement and
the reference's own known-answer tests; the C ABI's error paths that need no GPU."""

import ctypes
import os
import re

import numpy as np
import pytest

import julia_hip as jh
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "julia_hip.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    declared = set(re.findall(r"\b(julia_(?:cuda|hip)_\w+)\s*\(", header))
    assert declared == set(jh.EXPORTS), declared ^ set(jh.EXPORTS)
    L = jh.lib()
    for name in declared:
        assert getattr(L, name) is not None


def test_tier():
    assert jh.tier() == "gfx950"


def test_load_without_a_gpu_or_model_is_an_error():
    # A bad model spec fails before any device work; a good one fails on the GPU check here.
    with pytest.raises(jh.JuliaHipError, match="unknown model spec key"):
        jh.Engine("synthetic:bogus=1")
    with pytest.raises(jh.JuliaHipError, match="no model at"):
        jh.Engine("/some/checkpoint/dir")
    with pytest.raises(jh.JuliaHipError, match="d must be"):
        jh.Engine("synthetic:d=100")
    with pytest.raises(jh.JuliaHipError, match="batch_rows"):
        jh.Engine("synthetic:batch_rows=-1")
    # julia_hip_load's own batch_rows, checked before any device work
    with pytest.raises(jh.JuliaHipError, match="batch_rows out of range"):
        jh.Engine("synthetic", batch_rows=(1 << 20) + 1)
    if jh.device_count() == 0:
        with pytest.raises(jh.JuliaHipError, match="no HIP device"):
            jh.Engine("synthetic:layers=1")


def test_null_engine_and_free():
    L = jh.lib()
    L.julia_cuda_free(None)  # NULL is fine (src/capi.rs:91-96)
    err = ctypes.create_string_buffer(64)
    rc = L.julia_cuda_run(None, 1, None, None, None, None, None, 0, None, None, err, 64)
    assert rc == -1 and b"no engine" in err.value
    # the message is truncated to the buffer and NUL-terminated (src/capi.rs:23-33)
    err = ctypes.create_string_buffer(4)
    rc = L.julia_cuda_run(None, 1, None, None, None, None, None, 0, None, None, err, 4)
    assert rc == -1 and err.value == b"no "


@pytest.mark.parametrize("tid", [O.TOK_EMB, O.EMB_NORM, O.TYPE_EMB, O.LAYER_BASE + 1,
                                 O.LAYER_BASE + 16 * 21 + 4, O.HEAD_BASE + 32 + 7,
                                 O.SCORER_BASE + 5])
def test_synthetic_generator_matches_the_oracle(tid):
    mean, std = O.dist(tid)
    a = jh.synth(42, tid, 4099, mean, std, start=12345)
    b = O.synth(42, tid, 4099, start=12345)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # moments of the stream
    big = jh.synth(1, tid, 200000, 0.0, 1.0)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000) * 10 ** rng.uniform(-9, 5, 100000),
                        [0.0, -0.0, 65504, 65519, 65520, 1e9, -1e9, 2 ** -25, 2 ** -24,
                         3 * 2 ** -25, 6e-8, np.inf, -np.inf]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(jh.round_f16(x), want)
    assert np.array_equal(O.to_f16_bits(x), want)


def test_fold_layernorm_matches_the_oracle():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((96, 128)) * 0.02).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    beta = (0.05 * rng.standard_normal(128)).astype(np.float32)
    b = (0.02 * rng.standard_normal(96)).astype(np.float32)
    a16, acs = jh.fold_layernorm(w, g)
    b16, bcs = O.fold_layernorm(w, g)
    assert np.array_equal(a16, b16) and np.array_equal(acs.view(np.uint32), bcs.view(np.uint32))
    a16, acs, ab = jh.fold_layernorm_bias(w, g, beta, b)
    b16, bcs, bb = O.fold_layernorm_bias(w, g, beta, b)
    assert np.array_equal(a16, b16) and np.array_equal(ab.view(np.uint32), bb.view(np.uint32))


def test_bias_fold_matches_layernorm_then_linear():
    """The reference's known-answer test src/prep.rs:279-314, restated: xorshift64 from
    0x9e3779b97f4a7c15, k = 64, out = 32, 5 rows of mean ~3; the folded form within 2e-2 of
    LayerNorm (with bias) then linear (with bias), in f64."""
    seed = [0x9E3779B97F4A7C15]
    M = (1 << 64) - 1

    def rnd():
        s = seed[0]
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        seed[0] = s
        return (s >> 40) / float(1 << 24) - 0.5

    k, out, rows = 64, 32, 5
    w = np.array([rnd() for _ in range(out * k)], np.float32).reshape(out, k)
    gb = [(1.0 + rnd(), rnd()) for _ in range(k)]
    gamma = np.array([g for g, _ in gb], np.float32)
    beta = np.array([b for _, b in gb], np.float32)
    b = np.array([rnd() for _ in range(out)], np.float32)
    x = np.array([3.0 + rnd() for _ in range(rows * k)], np.float32).reshape(rows, k)
    w16, cs, bias = jh.fold_layernorm_bias(w, gamma, beta, b)
    wf = O.f16_bits_to_f32(w16).astype(np.float64)
    for row in x.astype(np.float64):
        mean = row.mean()
        r = 1.0 / np.sqrt(((row - mean) ** 2).mean() + 1e-5)
        ln = (row - mean) * r * gamma + beta
        want = w.astype(np.float64) @ ln + b
        got = r * (wf @ row - mean * cs.astype(np.float64)) + bias
        assert np.max(np.abs(got - want)) < 2e-2


def test_geglu_interleave_matches_the_epilogue():
    """The interleave against this library's GeGLU epilogue, as src/prep.rs:248-274 checks the
    reference's against its own: the thread owning columns c0 + e and c0 + 32 + e (c0 = 4 (t % 8),
    e < 4) of 64-column group g reads the input of output column 32 g + c0 + e at the first and
    its gate at the second; every output column is produced once."""
    inter = 1152
    rows = jh.geglu_rows(inter)
    assert np.array_equal(rows, O.geglu_rows(inter))
    seen = np.zeros(inter, bool)
    for g in range(2 * inter // 64):
        for t in range(8):
            for e in range(4):
                c0 = 4 * t
                col = 32 * g + c0 + e
                assert rows[64 * g + c0 + e] == col
                assert rows[64 * g + 32 + c0 + e] == inter + col
                assert not seen[col]
                seen[col] = True
    assert seen.all()
    assert sorted(rows) == list(range(2 * inter))


def test_fragment_order_packing():
    """The GEMM weight layout: the library's packing equals the oracle's numpy restatement,
    unpacking inverts it, and sampled elements sit where the MFMA lane map puts them (lane l of
    16 x 16 x 32 fragment j holds row 16 j + l % 16, K values 8 (l / 16) .. + 7 of its unit)."""
    rng = np.random.default_rng(7)
    n, k = 192, 96
    w = rng.integers(0, 1 << 16, (n, k), dtype=np.uint16)
    p = jh.pack_frag(w)
    assert np.array_equal(p, O.pack_frag(w))
    assert np.array_equal(jh.unpack_frag(p, n, k), w)
    U = k // 32
    for _ in range(500):
        G, u, j, l, e = (int(rng.integers(0, x)) for x in (n // 64, U, 4, 64, 8))
        assert p[(((G * U + u) * 4 + j) * 64 + l) * 8 + e] == w[64 * G + 16 * j + l % 16,
                                                                  32 * u + 8 * (l // 16) + e]
    with pytest.raises(jh.JuliaHipError):
        jh.pack_frag(w[:100])


def test_rope_table_matches_the_oracle_and_closed_form():
    a = jh.rope_table(160000.0, 300)
    assert np.array_equal(a, O.rope_table(160000.0, 300))
    p = np.arange(300)[:, None].astype(np.float64)
    j = np.arange(32)[None, :]
    ang = p * 160000.0 ** (-2.0 * j / 64)
    assert np.max(np.abs(a[:, :, 0] - np.cos(ang))) < 1e-4
    assert np.max(np.abs(a[:, :, 1] - np.sin(ang))) < 1e-4


def test_plan_matches_the_2080ti_sweeps():
    """The reference's golden picks, src/forward.rs:812-823 (68 SMs x 2 blocks, inter 1152,
    its D = 384): gemm_plan at 72, 363 and 512 tokens."""
    d, inter = 384, 1152
    shapes = [(3 * d, d), (d, d), (2 * inter, d), (d, inter)]
    picks = lambda n: [jh.gemm_plan_2080ti(n, c, k, 68, 2) for c, k in shapes]
    assert picks(72) == [(32, 1), (32, 3), (32, 1), (32, 3)]
    assert picks(363) == [(64, 1), (32, 1), (64, 1), (64, 3)]
    assert picks(512) == [(64, 1), (32, 1), (64, 1), (32, 1)]


def test_reference_choose_rule():
    """src/gemm.rs:153-172 in closed form."""
    assert jh.gemm_choose_2080ti(72, 1152, 384, 68) == (32, 1)     # 36 x 3 tiles > 34
    assert jh.gemm_choose_2080ti(72, 384, 384, 68) == (32, 4)      # 6 x 3 = 18 tiles
    assert jh.gemm_choose_2080ti(300, 384, 384, 68) == (64, 4)
    assert jh.gemm_choose_2080ti(500, 384, 384, 68) == (128, 4)     # 6 x 4 = 24 tiles
    assert jh.gemm_choose_2080ti(500, 1152, 384, 68) == (128, 1)    # 18 x 4 = 72 tiles
    assert jh.gemm_choose_2080ti(72, 384, 256, 68) == (32, 2)      # 8 K steps: 8 / 3 = 2


@pytest.mark.parametrize("m", [1, 72, 293, 512, 1024, 4096, 18752])
@pytest.mark.parametrize("n,k", [(2304, 768), (768, 768), (768, 1152), (1536, 768)])
def test_chooser_picks_valid_configs(m, n, k):
    bm, sp = jh.gemm_choose(m, n, k, 256)
    assert bm in (16, 32, 48, 64, 128, 192, 256)
    if bm >= 128:
        assert n % (256 if bm == 192 else bm) == 0 and sp == 1
    else:
        assert 1 <= sp <= 4 and (k // 32) // (4 * sp) >= 2


# The encoder's and head's GEMM shapes at width d (inter 1152, head_ff 1536) with their epilogues.
def _model_gemms(d, inter=1152, ff=1536):
    return [(3 * d, d, "lnrope"), (d, d, "resstats"), (2 * inter, d, "lngeglu"),
            (d, inter, "resstats"), (3 * d, d, "lnbias"), (ff, d, "lnbiasrelu"),
            (d, ff, "biasresstats"), (d, d, "lnbiasgelu")]


@pytest.mark.parametrize("d", [384, 768, 1280, 2048])
def test_every_pick_passes_the_launch_checks(d):
    """gemm_choose's pick for every model GEMM (with its epilogue) at every row count passes the
    launcher's own precondition checks (src/gemm.rs:262-329): in particular the throughput tiles'
    LayerNorm limit (k <= 1024), which widths past 1024 reach."""
    base = 1 << 20  # 16-byte aligned stand-in addresses (the check does not dereference them)
    for m in list(range(1, 4097, 37)) + [8192, 18752, 20000]:
        for n, k, epi in _model_gemms(d):
            flags = jh.EPI[epi]
            kw = {}
            if flags & jh.EPI_LN:
                kw.update(stats_in=base + 64, colsum=base + 128)
            if flags & jh.EPI_ROPE:
                kw.update(rope=base + 192, rope_rows=m)
            if flags & jh.EPI_STATS:
                kw.update(stats_out=base + 256)
            if flags & jh.EPI_BIAS:
                kw.update(bias=base + 320)
            args = jh.gemm_args(flags, base, base + 4096, base + 8192, m, n, k, **kw)
            bm, sp = jh.gemm_choose(m, n, k, 256, flags)
            jh.gemm_check(args, bm, sp, ws_floats=1 << 30, counters=1 << 20)
            if flags & jh.EPI_LN and k > 1024:
                assert bm < 128, (m, n, k, epi, bm)


def test_gemm_check_rejects_what_the_kernels_do_not_take():
    base = 1 << 20
    ln = dict(stats_in=base + 64, colsum=base + 128)
    ok = jh.gemm_args("lngeglu", base, base + 4096, base + 8192, 4096, 2560, 1280, **ln)
    jh.gemm_check(ok, 64)
    with pytest.raises(jh.JuliaHipError, match="LayerNorm epilogues up to k = 1024"):
        jh.gemm_check(ok, 256)
    with pytest.raises(jh.JuliaHipError, match="not a multiple of 64"):
        jh.gemm_check(jh.gemm_args("resstats", base, base, base + 64, 8, 100, 64,
                                   stats_out=base + 256), 16)
    with pytest.raises(jh.JuliaHipError, match="16-byte aligned"):
        jh.gemm_check(jh.gemm_args("resstats", base + 2, base, base + 8192, 8, 64, 64,
                                   stats_out=base + 256), 16)
    with pytest.raises(jh.JuliaHipError, match="scratch is too small"):
        jh.gemm_check(jh.gemm_args("resstats", base, base + 4096, base + 8192, 64, 768, 768,
                                   stats_out=base + 256), 32, 2)
    # the throughput tiles split K too (a 128 x 128 tile's partial is 16384 floats a split),
    # down to two K steps a split
    wo = jh.gemm_args("resstats", base, base + 4096, base + 8192, 512, 768, 768, stats_out=base + 256)
    jh.gemm_check(wo, 128, 4, ws_floats=24 * 4 * 128 * 128, counters=24)
    with pytest.raises(jh.JuliaHipError, match="scratch is too small"):
        jh.gemm_check(wo, 128, 4, ws_floats=24 * 4 * 128 * 128 - 1, counters=24)
    with pytest.raises(jh.JuliaHipError, match="fewer than two K steps"):
        jh.gemm_check(jh.gemm_args("resstats", base, base + 4096, base + 8192, 512, 768, 128,
                                   stats_out=base + 256), 256, 3, ws_floats=1 << 24, counters=64)
    # The throughput tiles address a, w and c through buffer descriptors (32-bit offsets); a row
    # past m stores to offset 0xFFFFFF00, outside any output the check lets through.
    rope = dict(rope=base + 512, rope_rows=1 << 21)
    big = jh.gemm_args("rope", base, base + 4096, base + 8192, (0xFFFFFF00 // 2304) // 2, 2304, 768, **rope)
    jh.gemm_check(big, 256)
    jh.gemm_check(jh.gemm_args("rope", base, base + 4096, base + 8192, 0xFFFFFF00 // 2 // 2304 - 255,
                               2304, 768, **rope), 128)
    with pytest.raises(jh.JuliaHipError, match="a, w and outputs up to 4 GB"):
        jh.gemm_check(jh.gemm_args("rope", base, base + 4096, base + 8192, 0xFFFFFF00 // 2 // 2304 + 1,
                                   2304, 768, **rope), 256)
    jh.gemm_check(jh.gemm_args("rope", base, base + 4096, base + 8192, 0xFFFFFF00 // 2 // 2304 + 1,
                               2304, 768, **rope), 64)  # the latency tiles take full pointers
    # The engine's own epilogues (the score folded into the scorer's lin1, the head's gathered
    # marker rows) take arguments the per-op ABI does not carry: through it they are refused.
    lin1 = dict(stats_in=base + 64, colsum=base + 128, bias=base + 256)
    with pytest.raises(jh.JuliaHipError, match="score weights and logits"):
        jh.gemm_check(jh.gemm_args(jh.EPI["lnbiasgelu"] | 256, base, base + 4096, base + 8192, 6,
                                   768, 768, **lin1), 16)
    with pytest.raises(jh.JuliaHipError, match="gathered rows"):
        jh.gemm_check(jh.gemm_args(jh.EPI["biasresstats"] | 512, base, base + 4096, base + 8192, 6,
                                   768, 768, bias=base + 256, stats_out=base + 512), 16)


@pytest.mark.parametrize("bm,pass_rows", [(16, 32), (32, 32), (48, 64), (64, 64)])
def test_split_scratch_covers_the_latency_tiles_partials(bm, pass_rows):
    """A split latency tile runs on four waves (256 threads, 8 a row), so its epilogue passes
    cover 32 rows and each split stores whole passes: ceil(bm / 32) passes x 2 halves x 256
    threads x 4 floats. The check accepts exactly that much scratch and no less."""
    base = 1 << 20
    ln = dict(stats_in=base + 64, colsum=base + 128)
    for m, n, k, splits in ((1536, 2304, 768, 2), (293, 2304, 768, 4), (512, 768, 1152, 3)):
        args = jh.gemm_args("lngeglu", base, base + 4096, base + 8192, m, n, k, **ln)
        tiles = (n // 64) * ((m + bm - 1) // bm)
        npass = (bm + 31) // 32
        need = tiles * splits * npass * 2 * 256 * 4
        assert need == tiles * splits * pass_rows * 64
        jh.gemm_check(args, bm, splits, ws_floats=need, counters=tiles)
        with pytest.raises(jh.JuliaHipError, match="scratch is too small"):
            jh.gemm_check(args, bm, splits, ws_floats=need - 1, counters=tiles)
    # The shape that exposed the 48-row under-count: 1152 tiles x 2 splits x 64 x 64 floats.
    big48 = jh.gemm_args("lngeglu", base, base + 4096, base + 8192, 1536, 2304, 768, **ln)
    with pytest.raises(jh.JuliaHipError, match="scratch is too small"):
        jh.gemm_check(big48, 48, 2, ws_floats=9_437_184 - 1, counters=1152)
    jh.gemm_check(big48, 48, 2, ws_floats=9_437_184, counters=1152)


def test_chooser_matches_the_measured_winners():
    """The picks at the shapes measured on MI355X (per-step GEMM times, the fastest config within
    a few percent): qkv/wi 48-row latency tiles at 293 tokens, wo and wo_mlp 16 rows."""
    assert jh.gemm_choose(293, 2304, 768, 256)[0] == 48
    assert jh.gemm_choose(293, 768, 768, 256)[0] == 16
    assert jh.gemm_choose(293, 768, 1152, 256)[0] == 16
    assert jh.gemm_choose(448, 768, 768, 256)[0] == 32
    # 448 tokens: 64-row tiles for qkv (252 tiles, the eight-wave kernel: 6.7 us against 10.4-12.0
    # for 16/32/48 and 10.5 for 128 x 128); 800: 128 x 128 for qkv (10.7 us against 12.3 for the
    # 64-row latency tiles), latency tiles for wo and wo_mlp (5.6 and 6.8 us on 48 rows against
    # 9.5 and 12.0 on 128 x 128)
    assert jh.gemm_choose(448, 2304, 768, 256)[0] == 64
    assert jh.gemm_choose(800, 2304, 768, 256) == (128, 1)
    assert jh.gemm_choose(800, 768, 768, 256)[0] == 48
    assert jh.gemm_choose(800, 768, 1152, 256)[0] == 48
    assert jh.gemm_choose(18752, 2304, 768, 256) == (256, 1)
    assert jh.gemm_choose(4096, 768, 768, 256) == (128, 1)
    assert jh.gemm_choose(18752, 768, 768, 256) == (256, 1)
    # the throughput tiles' models (a sweep of M = 2048 .. 18752 over the three tiles): 128 x 128
    # for qkv at 2048 and 8192 tokens (288 and 1152 tiles, two a CU), 192 x 256 at 4096 (198
    # tiles, one round: 24.4 us against 26.2 for 144 256 x 256 tiles and 27.6 for 128 x 128),
    # 256 x 256 at 6144 and 12288; 128 x 128 for wo at 2048-8192 (one tile a CU: 10.1 us
    # against 11.7 for the latency tiles at 2048)
    assert jh.gemm_choose(2048, 2304, 768, 256) == (128, 1)
    assert jh.gemm_choose(8192, 2304, 768, 256) == (128, 1)
    assert jh.gemm_choose(4096, 2304, 768, 256) == (192, 1)
    assert jh.gemm_choose(6144, 2304, 768, 256) == (256, 1)
    assert jh.gemm_choose(12288, 2304, 768, 256) == (256, 1)
    assert jh.gemm_choose(2048, 768, 768, 256) == (128, 1)
    assert jh.gemm_choose(8192, 768, 768, 256) == (128, 1)


def test_profiler_detection():
    """The measurement tools refuse cooperative launches under rocprofv3: its tool library in
    LD_PRELOAD or its ROCP_* / ROCPROF_* settings mark a profiled process."""
    assert jh.profiler_attached({}) is None
    assert jh.profiler_attached({"LD_PRELOAD": "/usr/lib/libfoo.so", "ROCM_PATH": "/opt/rocm"}) is None
    assert "LD_PRELOAD" in jh.profiler_attached(
        {"LD_PRELOAD": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"})
    assert "ROCP_TOOL_LIBRARIES" in jh.profiler_attached({"ROCP_TOOL_LIBRARIES": "x"})
    assert "ROCPROF_KERNEL_TRACE" in jh.profiler_attached({"ROCPROF_KERNEL_TRACE": "1"})


def test_kernel_trace_pairs_bench_runs_with_dispatches():
    """kernel_trace.py: each labelled run is the next stretch of its kernel at least warm-up +
    timed long (a set-up launch of the same kernel just before it merges into the stretch; only
    the last `timed` count), other kernels in between are skipped."""
    import kernel_trace as kt
    ds = [("void jh::gemm_big<256, 9, false>(GemmParams)", 50.0)]  # set-up launch, same name
    ds += [("void jh::gemm_big<256, 9, false>(GemmParams)", 40.0)] * 3  # warm-up
    ds += [("void jh::gemm_big<256, 9, false>(GemmParams)", 30.0 + i) for i in range(4)]
    ds += [("jh::embed_kernel", 5.0)] * 9
    ds += [("void jh::gemm_lat1<48, 20>(GemmParams)", 7.0)] * 2 + [("void jh::gemm_lat1<48, 20>(GemmParams)", 6.0)] * 4
    labels = [{"label": "wo@4096", "kernel": "gemm_big<256, 9, false>", "warmup": 3, "timed": 4},
              {"label": "qkv@293", "kernel": "gemm_lat1<48, 20>", "warmup": 2, "timed": 4}]
    runs = kt.pair(ds, labels)
    assert runs["wo@4096"]["launches"] == 4 and runs["wo@4096"]["avg_us"] == 31.5
    assert runs["wo@4096"]["min_us"] == 30.0 and runs["wo@4096"]["max_us"] == 33.0
    assert runs["qkv@293"]["avg_us"] == 6.0
    with pytest.raises(SystemExit):
        kt.pair(ds, labels + [{"label": "x", "kernel": "gemm_big", "warmup": 1, "timed": 1}])
