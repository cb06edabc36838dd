"""julia_hip_gemm_static, the GEMM entry point that allocates nothing (split-K partials and
counters in the library's static device scratch), through the C ABI: bit-identical to
julia_hip_gemm with a caller's scratch on the same inputs, over two calls in a row per shape
(the second smaller, so stale partials and counters of the first would show), and rejected with
the sizes when a tiling needs more scratch than the library holds."""

import numpy as np
import pytest

import julia_hip as jh
import oracle as O
from checks import EMU_REL, compare, f32, rand16
from conftest import f16_bits, to_dev

pytestmark = pytest.mark.gpu

EPS = 1e-5


def problem(kind, m, n, k, seed):
    rng = np.random.default_rng(seed)
    P = dict(kind=kind, epi=jh.EPI[kind], m=m, n=n, k=k, a=rand16(rng, (m, k), mean=0.1))
    W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if kind == "resstats":
        P["w"] = O.to_f16_bits(W)
        P["res"] = rand16(rng, (m, n))
        P["emu"], _ = O.emu_gemm(P["a"], P["w"], P["epi"], c16=P["res"])
    else:
        gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        P["w"], P["colsum"] = O.fold_layernorm(W, gamma)
        P["stats_in"] = O.row_stats(P["a"])
        if kind == "lnrope":
            P["rope"] = O.rope_table(160000.0, m)
        P["emu"] = O.emu_gemm(P["a"], P["w"], P["epi"], stats_in=P["stats_in"],
                              colsum=P["colsum"], eps=EPS, rope=P.get("rope"),
                              rope_cols=2 * n // 3 if kind == "lnrope" else 0)
    return P


def run(torch, P, bm, splits, scratch):
    """One launch: through julia_hip_gemm with `scratch`, or julia_hip_gemm_static (None)."""
    m, n, k = P["m"], P["n"], P["k"]
    dev = {key: to_dev(torch, P[key]) for key in ("a", "stats_in", "colsum", "rope") if key in P}
    dev["w"] = to_dev(torch, O.pack_frag(P["w"]))
    ncols = n // 2 if P["kind"] == "lngeglu" else n
    c = to_dev(torch, P["res"]) if "res" in P else torch.zeros((m, ncols), dtype=torch.float16,
                                                               device="cuda")
    st = torch.zeros((m, n // 64, 2), dtype=torch.float32, device="cuda") if "res" in P else None
    ptr = lambda key: dev[key].data_ptr() if key in dev else 0
    args = jh.gemm_args(P["epi"], ptr("a"), ptr("w"), c.data_ptr(), m, n, k,
                        stats_in=ptr("stats_in"), colsum=ptr("colsum"), eps=EPS, rope=ptr("rope"),
                        rope_rows=m, stats_out=st.data_ptr() if st is not None else 0)
    stream = torch.cuda.current_stream().cuda_stream
    if scratch is None:
        jh.gemm_static(args, bm=bm, splits=splits, stream=stream)
    else:
        jh.gemm(args, bm=bm, splits=splits, scratch=scratch, stream=stream)
    torch.cuda.synchronize()
    return f16_bits(c), (st.cpu().numpy() if st is not None else None)


# (kind, n, k, bm, splits, first m, second m): every split count the latency tiles take, the
# throughput tiles' K split (128 x 128 and 192 x 256), and the chooser's pick (bm 0).
CASES = [("resstats", 768, 1152, 32, 4, 512, 200), ("lngeglu", 2304, 768, 48, 2, 448, 100),
         ("lnrope", 2304, 768, 16, 3, 293, 72), ("resstats", 768, 768, 64, 2, 1024, 333),
         ("resstats", 768, 1152, 128, 2, 1100, 600), ("lngeglu", 2304, 768, 192, 2, 1000, 400),
         ("lnrope", 2304, 768, 0, 1, 293, 72)]


@pytest.mark.parametrize("kind,n,k,bm,splits,m1,m2", CASES)
def test_gemm_static_matches_gemm(torch_cuda, kind, n, k, bm, splits, m1, m2):
    scratch = jh.Scratch(ws_floats=1 << 24, counters=1 << 16)
    try:
        for call, m in enumerate((m1, m2)):
            print(f"gemm_static {kind} m={m} n={n} k={k} bm={bm} splits={splits} call {call}",
                  flush=True)
            P = problem(kind, m, n, k, seed=100 * call + n + k + m)
            want, want_st = run(torch_cuda, P, bm, splits, scratch)
            got, got_st = run(torch_cuda, P, bm, splits, None)
            assert np.array_equal(got, want), f"{kind} m={m}: output differs from julia_hip_gemm"
            if want_st is not None:
                assert np.array_equal(got_st.view(np.uint32), want_st.view(np.uint32))
            compare(f32(got), f32(P["emu"]), EMU_REL, what=f"{kind} m={m} vs emulation")
    finally:
        scratch.close()


def test_gemm_static_rejects_tilings_past_its_scratch(torch_cuda):
    torch = torch_cuda
    m, n, k = 8192, 2304, 768  # 16-row tiles, split 4: 18432 tiles > 16384 counters
    a = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    w = torch.zeros((n * k,), dtype=torch.float16, device="cuda")
    c = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    st = torch.zeros((m, n // 64, 2), dtype=torch.float32, device="cuda")
    args = jh.gemm_args("resstats", a.data_ptr(), w.data_ptr(), c.data_ptr(), m, n, k,
                        stats_out=st.data_ptr())
    with pytest.raises(jh.JuliaHipError, match="static scratch holds"):
        jh.gemm_static(args, bm=16, splits=4)
    # the same shape without a split takes no scratch and runs
    jh.gemm_static(args, bm=64, splits=1, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert float(c.float().abs().max()) == 0.0


def _operands(torch, m, n, k, seed):
    """LayerNorm-GeGLU operands on the device (the output is c alone, no residual)."""
    rng = np.random.default_rng(seed)
    a = rand16(rng, (m, k), mean=0.1)
    W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    w, colsum = O.fold_layernorm(W, gamma)
    dev = dict(a=to_dev(torch, a), w=to_dev(torch, O.pack_frag(w)), colsum=to_dev(torch, colsum),
               stats_in=to_dev(torch, O.row_stats(a)))
    dev["c"] = torch.zeros((m, n // 2), dtype=torch.float16, device="cuda")
    dev["args"] = jh.gemm_args("lngeglu", dev["a"].data_ptr(), dev["w"].data_ptr(),
                               dev["c"].data_ptr(), m, n, k, stats_in=dev["stats_in"].data_ptr(),
                               colsum=dev["colsum"].data_ptr(), eps=EPS)
    return dev


# (bm, the most rows whose two-way split fits the static scratch at n = 2304): a split latency
# tile stores whole 32-row passes (16 -> 32 rows, 48 -> 64), a throughput tile its BM x BN.
LIMITS = [(16, 896), (32, 1792), (48, 1344), (64, 1792), (128, 1792), (192, 1728), (256, 1792)]


@pytest.mark.parametrize("bm,m_max", LIMITS)
def test_gemm_static_at_its_scratch_limit(torch_cuda, bm, m_max):
    """The largest two-way split the static scratch holds runs and equals julia_hip_gemm bit for
    bit; one row more is refused before any launch."""
    torch = torch_cuda
    n, k = 2304, 768
    print(f"gemm_static limit bm={bm} m={m_max} (and {m_max + 1} refused)", flush=True)
    dev = _operands(torch, m_max + 1, n, k, seed=bm)
    over = jh.gemm_args("lngeglu", dev["a"].data_ptr(), dev["w"].data_ptr(), dev["c"].data_ptr(),
                        m_max + 1, n, k, stats_in=dev["stats_in"].data_ptr(),
                        colsum=dev["colsum"].data_ptr(), eps=EPS)
    with pytest.raises(jh.JuliaHipError, match="static scratch holds"):
        jh.gemm_static(over, bm=bm, splits=2)
    fit = jh.gemm_args("lngeglu", dev["a"].data_ptr(), dev["w"].data_ptr(), dev["c"].data_ptr(),
                       m_max, n, k, stats_in=dev["stats_in"].data_ptr(),
                       colsum=dev["colsum"].data_ptr(), eps=EPS)
    stream = torch.cuda.current_stream().cuda_stream
    scratch = jh.Scratch(ws_floats=1 << 24, counters=1 << 16)
    try:
        jh.gemm(fit, bm=bm, splits=2, scratch=scratch, stream=stream)
        torch.cuda.synchronize()
        want = f16_bits(dev["c"]).copy()
        dev["c"].zero_()
        jh.gemm_static(fit, bm=bm, splits=2, stream=stream)
        torch.cuda.synchronize()
        assert np.array_equal(f16_bits(dev["c"]), want), f"bm={bm} m={m_max}: differs from julia_hip_gemm"
    finally:
        scratch.close()


@pytest.mark.parametrize("bm,splits,m", [(48, 2, 448), (16, 3, 293), (128, 2, 1100)])
def test_gemm_static_under_graph_capture(torch_cuda, bm, splits, m):
    """julia_hip_gemm_static captured into a HIP graph (its counter-clearing kernel and the split
    GEMM), replayed three times with eager work and synchronisations in between: every replay
    equals julia_hip_gemm's output bit for bit."""
    torch = torch_cuda
    n, k = 2304, 768
    print(f"gemm_static graph bm={bm} splits={splits} m={m}", flush=True)
    dev = _operands(torch, m, n, k, seed=m)
    scratch = jh.Scratch(ws_floats=1 << 24, counters=1 << 16)
    try:
        stream = torch.cuda.current_stream().cuda_stream
        jh.gemm(dev["args"], bm=bm, splits=splits, scratch=scratch, stream=stream)
        torch.cuda.synchronize()
        want = f16_bits(dev["c"]).copy()
        # The first call on a device looks up the static array's address and sets kernel
        # attributes; it runs before the capture.
        jh.gemm_static(dev["args"], bm=bm, splits=splits, stream=stream)
        torch.cuda.synchronize()
        assert np.array_equal(f16_bits(dev["c"]), want)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                jh.gemm_static(dev["args"], bm=bm, splits=splits,
                               stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for replay in range(3):
            # eager work between the replays: the same GEMM through julia_hip_gemm, then c cleared
            jh.gemm(dev["args"], bm=bm, splits=splits, scratch=scratch, stream=stream)
            dev["c"].zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(f16_bits(dev["c"]), want), f"replay {replay} differs"
        graph.reset()
    finally:
        scratch.close()
