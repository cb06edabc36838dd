"""Multi-request throughput: julia_hip_run_batched packs consecutive requests into passes over
their concatenated rows (the varlen batching beyond the reference's one-by-one queue,
src/engine.rs:170-196). Every request's logits must equal what it gets alone through
julia_cuda_run (within the GEMMs' summation-order differences) and the f32 oracle's; the
packing, the shared pass times, the error paths and repeated markers are checked too."""

import numpy as np
import pytest

import julia_hip as jh
import oracle as O
from checks import check_logits

pytestmark = pytest.mark.gpu

SMALL = dict(d=384, layers=4, inter=1152, vocab=1000, head_ff=768, max_positions=2048, seed=7)
ROWS = 1500  # rows of one pass: 24 requests of up to 300 tokens take several passes
# Batched against one-by-one: the same f16 rounding points, only the GEMM tiles (and so the
# order of the K sums) differ with the rows (measured: mean |d| ~3e-5, max ~1.3e-4). Tight
# enough that a row given another question type fails (types differ by >= 2e-3 here).
PATH_MEAN, PATH_MAX = 1.5e-4, 5e-4


def spec(c):
    return "synthetic:" + ",".join(f"{k}={v}" for k, v in c.items())


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def engine(torch_cuda):
    say("engine: small synthetic model, batch rows", ROWS, spec(SMALL))
    e = jh.Engine(spec(SMALL), max_length=1024, batch_rows=ROWS)
    m = O.Model(O.cfg(**SMALL))
    yield e, m
    e.close()


def requests(rng, count, lo=1, hi=300):
    out = []
    for i in range(count):
        n = int(rng.integers(lo, hi))
        ids = rng.integers(0, SMALL["vocab"], n).astype(np.uint32)
        nm = int(rng.integers(0, 6))
        markers = rng.integers(0, n, nm).astype(np.uint32)  # repeats allowed, any order
        out.append((ids, markers, int(rng.integers(0, 3))))
    out[3] = (out[3][0][:1], np.zeros(2, np.uint32), 1)  # a one-token request
    return out


def passes(reqs, rows):
    """The packing julia_hip_run_batched does: consecutive requests while the rows fit."""
    out, cur, n = [], [], 0
    for i, r in enumerate(reqs):
        if cur and n + len(r[0]) > rows:
            out.append(cur)
            cur, n = [], 0
        cur.append(i)
        n += len(r[0])
    return out + [cur]


def path_diff(a, b, what):
    a, b = np.concatenate([np.asarray(x) for x in a]), np.concatenate([np.asarray(x) for x in b])
    assert a.shape == b.shape and np.isfinite(a).all(), what
    d = np.abs(a.astype(np.float64) - b)
    say(f"  {what}: {len(a)} logits, mean |d| {d.mean():.2e} max {d.max():.2e}")
    assert d.mean() <= PATH_MEAN and d.max() <= PATH_MAX, what


@pytest.mark.parametrize("fused", [False, True])
def test_batched_matches_one_by_one(engine, fused):
    e, m = engine
    rng = np.random.default_rng(21 + fused)
    reqs = requests(rng, 24)
    say(f"batched run: {len(reqs)} requests, {sum(len(r[0]) for r in reqs)} rows, fused={fused}")
    if fused:  # the passes run as whole-model launches
        assert all(e.model_kernel(sum(len(reqs[i][0]) for i in g)) for g in passes(reqs, ROWS))
    got, ms = e.run(reqs, layer_fused=fused, batched=True)
    alone, _ = e.run(reqs, layer_fused=fused)
    path_diff(got, alone, "batched vs julia_cuda_run")
    # every request of a pass has that pass's time; the passes are the greedy packing
    groups = passes(reqs, ROWS)
    assert len(groups) >= 3
    for g in groups:
        assert np.all(ms[g] == ms[g[0]]) and ms[g[0]] > 0
    for i in range(0, len(reqs), 5):
        ids, markers, q = reqs[i]
        if len(markers):
            check_logits(got[i], m.forward(ids, q, markers), f"request {i} against the oracle")


def test_batched_one_pass_and_single_request(engine):
    """Everything in one pass (rows well under the limit), and one request alone: the batched
    path's logits for a lone request are julia_cuda_run's within the path tolerance. The same
    tokens under the three question types in one pass: each row adds its own type's embedding
    (the logits differ by type, each as one by one)."""
    e, _ = engine
    rng = np.random.default_rng(5)
    reqs = requests(rng, 6, 40, 200)
    got, ms = e.run(reqs, batched=True)
    assert np.all(ms == ms[0])
    alone, _ = e.run(reqs)
    path_diff(got, alone, "one pass")
    k = next(i for i, r in enumerate(reqs) if len(r[1]))
    one, _ = e.run(reqs[k:k + 1], batched=True)
    path_diff(one, alone[k:k + 1], "single request")
    ids = rng.integers(0, SMALL["vocab"], 120).astype(np.uint32)
    typed = [(ids, np.array([0, 60, 119], np.uint32), q) for q in (0, 1, 2)]
    got, _ = e.run(typed, batched=True)
    alone, _ = e.run(typed)
    path_diff(got, alone, "question types")
    for a in range(3):
        for b in range(a):
            assert np.abs(got[a] - got[b]).max() > 2 * PATH_MAX, (a, b, got)


def test_full_pass_of_max_length_requests(engine):
    """Requests at max_length that exactly fill passes (1024 + 476 = 1500 rows)."""
    e, _ = engine
    rng = np.random.default_rng(8)
    reqs = []
    for n in (1024, 476, 1024, 476):
        ids = rng.integers(0, SMALL["vocab"], n).astype(np.uint32)
        reqs.append((ids, np.array([0, n // 2, n - 1], np.uint32), n % 3))
    got, ms = e.run(reqs, batched=True)
    assert ms[0] == ms[1] and ms[2] == ms[3]
    alone, _ = e.run(reqs)
    path_diff(got, alone, "full passes")


def test_many_markers(engine):
    """A request may name a marker any number of times (src/engine.rs:78-81 only bounds the
    positions): more markers than max_length, through the graph path, the direct path and the
    batched path; repeated markers give identical logits. (With more markers than rows the head
    runs on every row and the score kernel sums each logit; with fewer, on the marker rows with
    the score summed in lin1's epilogue: the same values up to the order of the f32 sums.)"""
    e, _ = engine
    rng = np.random.default_rng(11)
    ids = rng.integers(0, SMALL["vocab"], 50).astype(np.uint32)
    # 18000 markers: past max_length and past the 16 x max_length the engine starts with
    markers = np.tile(np.array([3, 17, 49], np.uint32), 6000)
    small = (ids, np.array([3, 17, 49], np.uint32), 2)
    for fused, batched in ((False, False), (True, False), (False, True)):
        out, _ = e.run([small, (ids, markers, 2), small], layer_fused=fused, batched=batched)
        assert len(out[1]) == 18000
        np.testing.assert_array_equal(out[1].reshape(6000, 3), np.tile(out[1][:3], (6000, 1)))
        if batched:  # the same request at another row offset: key blocks fall differently
            path_diff([out[1][:3], out[2]], [out[0], out[0]], "repeated request, batched")
        else:
            np.testing.assert_allclose(out[1][:3], out[0], rtol=0, atol=1e-6)
            np.testing.assert_array_equal(out[2], out[0])


def test_batched_errors(engine):
    """julia_cuda_run's checks, through the batched entry point: -1 and a message, nothing run."""
    e, _ = engine
    ids = np.arange(10, dtype=np.uint32)
    good = (ids, [1], 0)
    for bad, match in (((ids, [1], 3), "question type"), ((ids, [10], 0), "marker is past"),
                       ((np.zeros(0, np.uint32), [], 0), "tokens, not 1 to"),
                       ((np.zeros(1025, np.uint32), [], 0), "tokens, not 1 to"),
                       ((np.array([5, 1000], np.uint32), [0], 0), "vocabulary")):
        with pytest.raises(jh.JuliaHipError, match=match):
            e.run([good, bad], batched=True)
    out, _ = e.run([good, (ids, [3], 0)], batched=True)
    assert np.isfinite(out[1]).all()


def test_batch_rows_bounds(torch_cuda):
    with pytest.raises(jh.JuliaHipError, match="batch_rows"):
        jh.Engine(spec(SMALL), max_length=64, batch_rows=(1 << 20) + 1)
    # batch_rows below max_length: every pass still holds a max_length request
    e = jh.Engine(spec(SMALL), max_length=256, batch_rows=100)
    rng = np.random.default_rng(2)
    reqs = [(rng.integers(0, 1000, n).astype(np.uint32), [0, n - 1], 0) for n in (256, 30, 200)]
    got, ms = e.run(reqs, batched=True)
    alone, _ = e.run(reqs)
    path_diff(got, alone, "batch_rows under max_length")
    e.close()


def test_marker_rows_on_throughput_tiles(torch_cuda):
    """A pass with thousands of marker rows (fewer than its rows): the chooser gives the head's
    marker-row GEMMs throughput tiles, which neither gather rows nor carry the score, so a gather
    kernel and the score kernel run; with a few hundred markers the GEMMs gather and score
    themselves. Both against each request alone and the oracle."""
    e = jh.Engine(spec(SMALL), max_length=1024, batch_rows=4096)
    m = O.Model(O.cfg(**SMALL))
    rng = np.random.default_rng(17)
    for nm in (700, 90):  # 4 x 700 = 2800 marker rows: 128-row tiles; 4 x 90: latency tiles
        assert jh.gemm_choose(4 * nm, SMALL["d"], SMALL["d"], 256, 164)[0] == (128 if nm == 700 else 16)
        reqs = []
        for i in range(4):
            ids = rng.integers(0, SMALL["vocab"], 1000).astype(np.uint32)
            reqs.append((ids, rng.integers(0, 1000, nm).astype(np.uint32), i % 3))
        got, ms = e.run(reqs, batched=True)
        assert np.all(ms == ms[0])
        alone, _ = e.run(reqs)
        path_diff(got, alone, f"{4 * nm} marker rows in one pass")
        ids, markers, q = reqs[1]
        check_logits(got[1][:8], m.forward(ids, q, markers[:8]), f"{4 * nm} marker rows, oracle")
    e.close()
