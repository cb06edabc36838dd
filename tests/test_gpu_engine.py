"""The whole forward pass through the drop-in C ABI (julia_cuda_load / julia_cuda_run), against
the CPU oracle's f32 forward on the same seeded synthetic model: the reference's --check flow
(src/main.rs:180-232) as tests: the weight upload (bit-exact against the oracle's own
preparation), each encoder layer's residual stream, the head and the logits, per-step kernels
and the persistent layer kernel, and the C ABI's error paths (src/capi.rs, src/engine.rs)."""

import numpy as np
import pytest

import julia_hip as jh
import oracle as O
from checks import check_logits, compare, f32

pytestmark = pytest.mark.gpu

SMALL = dict(d=384, layers=4, inter=1152, vocab=1000, head_ff=768, max_positions=2048, seed=7)
CHAINED_REL = 3e-2  # src/check.rs:395-402: the chain through all layers


def spec(c):
    return "synthetic:" + ",".join(f"{k}={v}" for k, v in c.items())


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def small(torch_cuda):
    say("engine: small synthetic model", spec(SMALL))
    e = jh.Engine(spec(SMALL), max_length=1024)
    m = O.Model(O.cfg(**SMALL))
    yield e, m
    e.close()


def request(rng, n, vocab, nm=4):
    ids = rng.integers(0, vocab, n).astype(np.uint32)
    markers = np.sort(rng.choice(n, size=min(nm, n), replace=False)).astype(np.uint32)
    return ids, markers


def test_tier_and_device(small):
    e, _ = small
    assert jh.tier() == "gfx950"
    say("device:", e.device())
    assert e.device()


def test_weights_match_the_oracle_preparation(small):
    """GpuWeights::verify (src/weights.rs:257-271), against an independent preparation."""
    e, m = small
    c = SMALL
    d, I = c["d"], c["inter"]
    seed = c["seed"]
    # layer 0: converted only; layer 1: folded; wi interleaved for GeGLU
    w0 = O.synth(seed, O.LAYER_BASE + O.L_WQKV, 3 * d * d).reshape(3 * d, d)
    assert np.array_equal(e.tensor_host("wqkv", 0), O.pack_frag(O.to_f16_bits(w0)))
    b = O.LAYER_BASE + 16
    w1 = O.synth(seed, b + O.L_WQKV, 3 * d * d).reshape(3 * d, d)
    g1 = O.synth(seed, b + O.L_ATTN_NORM, d)
    w16, cs = O.fold_layernorm(w1, g1)
    assert np.array_equal(e.tensor_host("wqkv", 1), O.pack_frag(w16))
    assert np.array_equal(e.tensor_host("qkv_colsum", 1, np.float32), cs)
    wi = O.synth(seed, b + O.L_WI, 2 * I * d).reshape(2 * I, d)
    gi = O.synth(seed, b + O.L_MLP_NORM, d)
    wi16, wcs = O.fold_layernorm(wi, gi)
    rows = O.geglu_rows(I)
    assert np.array_equal(e.tensor_host("wi", 1), O.pack_frag(wi16[rows]))
    assert np.array_equal(e.tensor_host("wi_colsum", 1, np.float32), wcs[rows])
    # the head's bias fold and the embedding table
    hb = O.HEAD_BASE + 32
    ip = O.synth(seed, hb + O.H_IN_PROJ_W, 3 * d * d).reshape(3 * d, d)
    _, _, ipb = O.fold_layernorm_bias(ip, O.synth(seed, hb + O.H_NORM1_W, d),
                                      O.synth(seed, hb + O.H_NORM1_B, d),
                                      O.synth(seed, hb + O.H_IN_PROJ_B, 3 * d))
    assert np.array_equal(e.tensor_host("in_proj_b", 1, np.float32), ipb)
    emb = e.tensor_host("tok_emb", 0)
    assert np.array_equal(emb[: 10 * d], O.to_f16_bits(O.synth(seed, O.TOK_EMB, 10 * d)))


@pytest.mark.parametrize("n", [72, 363])
def test_forward_matches_oracle(small, n):
    e, m = small
    say(f"forward n={n} (per-step kernels)")
    rng = np.random.default_rng(n)
    ids, markers = request(rng, n, SMALL["vocab"])
    want, trace = m.forward(ids, 0, markers, trace=True)
    logits, xt, _ = e.run_trace(ids, markers, 0)
    for layer in range(SMALL["layers"]):
        compare(f32(xt[layer]), trace[layer], CHAINED_REL, 1e-1, what=f"layer {layer} stream")
    mean, mx = check_logits(logits, want)
    say(f"  logits {np.round(logits, 4)} vs {np.round(want, 4)}: mean |d| {mean:.2e} max {mx:.2e}")
    # and through julia_cuda_run
    out, ms = e.run([(ids, markers, 0)])
    np.testing.assert_allclose(out[0], logits, rtol=0, atol=1e-6)
    assert ms[0] > 0


def test_layer_kernel_matches_per_step(small):
    """src/check.rs:665-760 `layer_kernel`: the persistent kernel against the per-step kernels
    (same tasks; summation order differs only in the split-K / key-range merges)."""
    e, m = small
    rng = np.random.default_rng(3)
    for n in (72, 363, 1000):
        say(f"layer kernel n={n}")
        ids, markers = request(rng, n, SMALL["vocab"])
        ls, xs, _ = e.run_trace(ids, markers, 1)
        lf, xf, _ = e.run_trace(ids, markers, 1, layer_fused=True)
        for layer in range(SMALL["layers"]):
            compare(f32(xf[layer]), f32(xs[layer]), 1e-2, 5e-2, what=f"fused layer {layer}")
        want = m.forward(ids, 1, markers)
        check_logits(lf, want, "layer kernel logits")


def test_whole_model_kernel(small):
    """layer_fused through julia_cuda_run: the whole forward pass as one cooperative launch
    (embed, the layers, the head, the score; the reference's stated next step, README.md:12-13),
    against the oracle and the per-step kernels, every question type, up to max_length."""
    e, m = small
    rng = np.random.default_rng(13)
    for n in (72, 363, 1024):
        assert e.model_kernel(n), n
        ids, markers = request(rng, n, SMALL["vocab"], nm=5)
        q = n % 3
        say(f"whole-model kernel n={n} qtype={q}")
        lf, ms = e.run([(ids, markers, q), (ids, markers, q)], layer_fused=True)
        ls, _ = e.run([(ids, markers, q)])
        np.testing.assert_array_equal(lf[0], lf[1])  # deterministic launch to launch
        d = np.abs(lf[0] - ls[0]).max()
        mean, mx = check_logits(lf[0], m.forward(ids, q, markers), "whole-model logits")
        say(f"  oracle mean |d| {mean:.2e} max {mx:.2e}; per-step max |d| {d:.2e}; {ms[0]:.3f} ms")
        assert d <= 1e-2
    assert not e.model_kernel(0) and not e.model_kernel(1025)


def test_no_head_layers(torch_cuda):
    """A model with no head layers (norm_add straight into the scorer): the per-step path, the
    whole-model launch and the batched pass against the oracle."""
    c = dict(SMALL, head_layers=0)
    e = jh.Engine(spec(c), max_length=512, batch_rows=1024)
    m = O.Model(O.cfg(**c))
    rng = np.random.default_rng(31)
    reqs = []
    for n in (40, 300, 129):
        ids, markers = request(rng, n, c["vocab"])
        reqs.append((ids, markers, n % 3))
    for fused in (False, True):
        for batched in (False, True):
            out, _ = e.run(reqs, layer_fused=fused, batched=batched)
            for (ids, markers, q), lg in zip(reqs, out):
                check_logits(lg, m.forward(ids, q, markers), f"fused={fused} batched={batched}")
    assert e.model_kernel(300)
    e.close()


def test_batch_of_requests(small):
    """Engine::run's queue (src/engine.rs:170-196): more requests than one queue of 16, mixed
    lengths and question types, against each request run alone."""
    e, m = small
    rng = np.random.default_rng(9)
    reqs = []
    for i in range(20):
        n = int(rng.integers(1, 300))
        ids, markers = request(rng, n, SMALL["vocab"], nm=int(rng.integers(0, 4)))
        reqs.append((ids, markers, i % 3))
    out, ms = e.run(reqs)
    assert len(out) == 20 and np.all(ms > 0)
    for (ids, markers, q), lg in list(zip(reqs, out))[::4]:
        alone, _ = e.run([(ids, markers, q)])
        np.testing.assert_allclose(lg, alone[0], rtol=0, atol=1e-6)
        if len(markers):
            check_logits(lg, m.forward(ids, q, markers))


def test_run_errors(small):
    """The C ABI's failures (src/capi.rs:157-168, src/engine.rs:78-81): -1 and a message."""
    e, _ = small
    ids = np.arange(10, dtype=np.uint32)
    with pytest.raises(jh.JuliaHipError, match="question type"):
        e.run([(ids, [1], 3)])
    with pytest.raises(jh.JuliaHipError, match="marker is past"):
        e.run([(ids, [10], 0)])
    with pytest.raises(jh.JuliaHipError, match="tokens, not 1 to"):
        e.run([(np.zeros(0, np.uint32), [], 0)])
    with pytest.raises(jh.JuliaHipError, match="tokens, not 1 to"):
        e.run([(np.zeros(1025, np.uint32), [], 0)])
    with pytest.raises(jh.JuliaHipError, match="vocabulary"):
        e.run([(np.array([5, 1000], np.uint32), [0], 0)])
    # the engine still works afterwards
    out, _ = e.run([(ids, [3], 0)])
    assert np.isfinite(out[0]).all()


@pytest.mark.parametrize("batched", [False, True])
def test_bad_request_past_the_first_queue_runs_nothing(small, batched):
    """src/capi.rs:150-170 checks every sequence before Engine::run: a bad request at index 16
    (past the first queue of 16) fails the call before any request has run, so the logits and
    times of the good requests before it are left as they were."""
    import ctypes
    e, _ = small
    rng = np.random.default_rng(16)
    reqs = [(rng.integers(0, SMALL["vocab"], 20).astype(np.uint32), np.array([1, 5], np.uint32), 0)
            for _ in range(20)]
    reqs[16] = (reqs[16][0], np.array([25], np.uint32), 0)  # marker past the sequence
    ids = np.concatenate([r[0] for r in reqs])
    lens = np.array([len(r[0]) for r in reqs], np.uintp)
    markers = np.concatenate([r[1] for r in reqs])
    nm = np.array([len(r[1]) for r in reqs], np.uintp)
    qt = np.zeros(len(reqs), np.uint32)
    logits = np.full(len(markers), -7.0, np.float32)
    ms = np.full(len(reqs), -7.0, np.float32)
    err = ctypes.create_string_buffer(256)
    fn = jh.lib().julia_hip_run_batched if batched else jh.lib().julia_cuda_run
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    rc = fn(e.ptr, len(reqs), p(ids), p(lens), p(markers), p(nm), p(qt), 0, p(logits), p(ms),
            err, 256)
    assert rc == -1 and b"marker is past" in err.value, err.value
    assert np.all(logits == -7.0) and np.all(ms == -7.0)


def test_batched_encoder_matches_each_request(torch_cuda):
    """Config 5's batched variant: requests concatenated into one set of rows,
    positions restarting in every request and attention kept within each, give every request its
    own encoder output: against the request run alone (per-step kernels) and against the f32
    oracle. The batch passes 2048 rows, so the per-step path takes the throughput GEMMs."""
    c = dict(SMALL, batch_rows=4096)
    e = jh.Engine(spec(c), max_length=1024)
    m = O.Model(O.cfg(**SMALL))
    rng = np.random.default_rng(21)
    lens = [70, 130, 45, 200, 17, 513, 300, 64, 97, 1, 256, 400, 300]
    seqs = [rng.integers(0, SMALL["vocab"], n).astype(np.uint32) for n in lens]
    assert sum(lens) > 2048
    alone = {i: e.run_trace(seqs[i], [], 0)[1][-1] for i in range(0, len(seqs), 3)}
    oracle = {i: m.forward(seqs[i], 0, [], trace=True)[1][-1] for i in (1, 5)}
    for fused in (False, True):
        x, ms = e.encode_batch(seqs, layer_fused=fused)
        say(f"batched encoder ({'layer kernel' if fused else 'per-step'}): {sum(lens)} rows, "
            f"{ms:.3f} GPU ms")
        assert ms > 0 and x.shape == (sum(lens), SMALL["d"])
        starts = np.concatenate([[0], np.cumsum(lens)])
        for i, want in alone.items():
            got = x[starts[i]:starts[i + 1]]
            compare(f32(got), f32(want), 1e-2, 5e-2, what=f"request {i} ({lens[i]} rows)")
        for i, want in oracle.items():
            got = x[starts[i]:starts[i + 1]]
            compare(f32(got), want, CHAINED_REL, 1e-1, what=f"request {i} vs oracle")
    with pytest.raises(jh.JuliaHipError, match="rows are over"):
        e.encode_batch([seqs[5]] * 8)
    with pytest.raises(jh.JuliaHipError, match="tokens, not 1 to"):
        e.encode_batch([np.zeros(1025, np.uint32)])
    e.close()


def test_batched_encoder_on_256_tiles(torch_cuda):
    """The persistent kernel's 256 x 256 instance (512-thread blocks, the streaming attention
    tile on eight waves): config 4's widths, a batch past 2048 rows; the layer kernel against
    the per-step kernels."""
    c = dict(d=768, layers=2, inter=1152, vocab=1000, head_ff=768, max_positions=4096, seed=11,
             batch_rows=2600)
    e = jh.Engine(spec(c), max_length=1024)
    plan, _ = e.profile_layer(2600, 0)
    assert list(plan[:4]) == [256, 256, 256, 256], plan
    rng = np.random.default_rng(23)
    lens = [300, 1024, 17, 700, 1, 513]
    seqs = [rng.integers(0, c["vocab"], n).astype(np.uint32) for n in lens]
    xs, _ = e.encode_batch(seqs, layer_fused=False)
    xf, ms = e.encode_batch(seqs, layer_fused=True)
    say(f"256-tile layer kernel: {sum(lens)} rows, {ms:.3f} GPU ms")
    compare(f32(xf), f32(xs), 1e-2, 5e-2, what="layer kernel vs per-step")
    e.close()


def test_whole_model_on_256_tiles(torch_cuda):
    """The whole-model launch on the 256 x 256 instance (config 4's widths, head_ff 1536, a
    batched pass past 2048 rows): every head GEMM on the throughput tile, attention bounded to
    each request, every question type; against the per-step kernels on the same pass and the
    oracle on single requests."""
    c = dict(d=768, layers=2, inter=1152, vocab=1000, head_ff=1536, max_positions=4096, seed=11)
    e = jh.Engine(spec(c), max_length=1024, batch_rows=2600)
    m = O.Model(O.cfg(**c))
    rng = np.random.default_rng(29)
    lens = [300, 1024, 17, 700, 1, 513]
    reqs = []
    for i, n in enumerate(lens):
        ids = rng.integers(0, c["vocab"], n).astype(np.uint32)
        reqs.append((ids, rng.integers(0, n, 4).astype(np.uint32), i % 3))
    assert e.model_kernel(sum(lens))
    plan, _ = e.profile_layer(sum(lens), 0)
    assert list(plan[:4]) == [256, 256, 256, 256], plan
    lf, ms = e.run(reqs, layer_fused=True, batched=True)
    ls, _ = e.run(reqs, batched=True)
    a, b = np.concatenate(lf), np.concatenate(ls)
    say(f"whole model, 256 tiles: {sum(lens)} rows {ms[0]:.3f} ms; max |d| to per-step "
        f"{np.abs(a - b).max():.2e}")
    assert np.isfinite(a).all() and np.abs(a - b).max() <= 1e-2
    for i in (0, 2, 5):
        ids, markers, q = reqs[i]
        check_logits(lf[i], m.forward(ids, q, markers), f"request {i} against the oracle")
    e.close()


def test_fused_fallback_when_the_head_does_not_fit(torch_cuda):
    """A head the 256 x 256 instance cannot take (head_ff 1152, not a multiple of 256): the
    layer_fused pass falls back to the encoder kernel and the head's own launches, and still
    matches the per-step kernels."""
    c = dict(d=768, layers=2, inter=1152, vocab=1000, head_ff=1152, max_positions=4096, seed=13)
    e = jh.Engine(spec(c), max_length=1024, batch_rows=2600)
    rng = np.random.default_rng(37)
    lens = [1024, 700, 513, 300]
    reqs = [(rng.integers(0, c["vocab"], n).astype(np.uint32),
             rng.integers(0, n, 3).astype(np.uint32), i % 3) for i, n in enumerate(lens)]
    plan, _ = e.profile_layer(sum(lens), 0)
    assert list(plan[:4]) == [256, 256, 256, 256], plan
    assert not e.model_kernel(sum(lens)) and e.model_kernel(300)
    lf, _ = e.run(reqs, layer_fused=True, batched=True)
    ls, _ = e.run(reqs, batched=True)
    a, b = np.concatenate(lf), np.concatenate(ls)
    say(f"fallback: max |d| to per-step {np.abs(a - b).max():.2e}")
    assert np.isfinite(a).all() and np.abs(a - b).max() <= 1e-2
    e.close()


def test_load_errors(torch_cuda):
    with pytest.raises(jh.JuliaHipError, match="max_length"):
        jh.Engine(spec(dict(SMALL, max_positions=512)), max_length=600)
    with pytest.raises(jh.JuliaHipError, match="no model"):
        jh.Engine("/no/such/checkpoint")


def test_full_model_293_tokens(torch_cuda):
    """Config 4's model (ModernBERT-base shapes, 22 layers, head_ff 1536) on one 293-token
    request: logits within the north star's tolerance of the f32 oracle."""
    say("full model d=768 layers=22 n=293")
    e = jh.Engine("synthetic", max_length=1024)
    try:
        m = O.Model(O.cfg())
        rng = np.random.default_rng(293)
        ids, markers = request(rng, 293, 50368, nm=6)
        want, trace = m.forward(ids, 0, markers, trace=True)
        logits, xt, _ = e.run_trace(ids, markers, 0)
        worst = max(O.rel_err(f32(xt[l]), trace[l]) for l in range(22))
        mean, mx = check_logits(logits, want)
        lf, _, _ = e.run_trace(ids, markers, 0, layer_fused=True, trace=False)
        check_logits(lf, want, "layer kernel")
        say(f"  worst layer stream rel err {worst:.2e}; logits mean |d| {mean:.2e} max {mx:.2e}")
        assert worst < CHAINED_REL
    finally:
        e.close()


def test_barrier_time_out_is_an_error_not_wrong_logits(torch_cuda, small, monkeypatch):
    """A persistent launch whose grid barriers never complete (forced from the host: every barrier
    waits for one generation more than its arrivals make, the state a grid that is not
    co-resident leaves) ends in the bounded wait's error, with every block run to its end; the
    barrier words are reset, so the same engine's next passes are right on both paths."""
    e_ok, m = small
    rng = np.random.default_rng(31)
    ids, markers = request(rng, 200, SMALL["vocab"])
    want, _ = e_ok.run([(ids, markers, 1)], layer_fused=True)
    monkeypatch.setenv("JULIA_HIP_TEST_BARRIER_SKEW", "1")
    say("engine: barrier skew (time-out path)", spec(SMALL))
    e = jh.Engine(spec(SMALL), max_length=1024)
    monkeypatch.delenv("JULIA_HIP_TEST_BARRIER_SKEW")
    try:
        with pytest.raises(jh.JuliaHipError, match="grid barrier timed out"):
            e.run([(ids, markers, 1)], layer_fused=True)
        got, _ = e.run([(ids, markers, 1)], layer_fused=False)
        check_logits(got[0], want[0], what="per-step after a barrier time-out")
    finally:
        e.close()
    again, _ = e_ok.run([(ids, markers, 1)], layer_fused=True)
    assert np.array_equal(again[0], want[0])
