"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it: each function
against something it shares no code with (library routines, closed forms, the committed golden
fixtures written by an independent torch restatement, brute force), chosen so that a plausible
mistake (a dropped scale, a wrong sign or pair, an off-by-one window, a transposed operand) fails.
Then the tests of the tests (src/check.rs:837-871, :1132-1184): the parity checks reject
known-wrong outputs, with the f16 emulation standing in for a correct kernel."""

import math
import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from checks import ATTN_REL, EMU_REL, GEMM_REL, check_stats, compare, f32, rand16

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import torch_reference as T  # noqa: E402

GOLD = os.path.join(HERE, "golden")


def test_f16_round_trip():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = (h & 0x7C00) != 0x7C00
    back = O.to_f16_bits(O.f16_bits_to_f32(h[finite]))
    assert np.array_equal(back, h[finite])
    assert np.array_equal(np.array([O.lib().oracle_f16_to_f32(int(v)) for v in h[::257]], np.float32),
                          h[::257].view(np.float16).astype(np.float32), equal_nan=True)


def test_gelu_is_erf_gelu_within_the_published_bound():
    g = np.load(os.path.join(GOLD, "ops.npz"))
    got = O.gelu(g["gelu_x"])
    # A&S 7.1.26: |erf error| <= 1.5e-7, so |GELU error| <= |x| * 0.75e-7, plus f32 rounding.
    bound = 0.75e-7 * np.abs(g["gelu_x"]) + 2e-7 * np.maximum(1, np.abs(g["gelu"]))
    assert np.all(np.abs(got - g["gelu"]) <= bound)
    assert O.gelu(np.array([0.0]))[0] == 0.0


def test_layernorm_against_torch():
    g = np.load(os.path.join(GOLD, "ops.npz"))
    got = O.layernorm_rows(g["ln_x"], g["ln_g"], g["ln_b"], 1e-5)
    np.testing.assert_allclose(got, g["ln"], rtol=1e-6, atol=1e-6)
    nob = O.layernorm_rows(g["ln_x"], g["ln_g"], None, 1e-5)
    np.testing.assert_allclose(nob, g["ln"] - g["ln_b"], rtol=1e-5, atol=1e-5)


def test_linear_against_numpy():
    rng = np.random.default_rng(1)
    x, w, b = rng.standard_normal((13, 70)), rng.standard_normal((33, 70)), rng.standard_normal(33)
    np.testing.assert_allclose(O.linear(x, w, b), x @ w.T + b, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.linear(x, w), x @ w.T, rtol=1e-5, atol=1e-5)


def test_rope_against_complex_rotation():
    g = np.load(os.path.join(GOLD, "ops.npz"))
    n = g["rope_x"].shape[0]
    qkv = np.zeros((n, 3 * 128), np.float32)
    qkv[:, :128] = g["rope_x"]
    qkv[:, 128:256] = g["rope_x"]
    qkv[:, 256:] = 7.0
    got = O.rope_apply(qkv, O.rope_table(10000.0, n))
    np.testing.assert_allclose(got[:, :128], g["rope"], atol=2e-5)
    np.testing.assert_allclose(got[:, 128:256], g["rope"], atol=2e-5)
    assert np.all(got[:, 256:] == 7.0)  # v is not rotated
    # position 0 is the identity; the rotation keeps each pair's norm
    assert np.allclose(got[0, :128], qkv[0, :128])
    pn = lambda a: a[:, :32] ** 2 + a[:, 32:64] ** 2
    np.testing.assert_allclose(pn(got[:, :128]), pn(qkv[:, :128]), rtol=1e-5)


@pytest.mark.parametrize("window", [0, 3])
def test_attention_against_torch_sdpa(window):
    g = np.load(os.path.join(GOLD, "ops.npz"))
    got = O.attention(g["qkv"], window)
    want = g["att_global" if window == 0 else "att_window3"]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_attention_brute_force_and_window_edge():
    """Keys outside the window have no effect; the boundary |i - j| == window is inside."""
    rng = np.random.default_rng(2)
    n, d, w = 9, 64, 2
    qkv = rng.standard_normal((n, 3 * d)).astype(np.float32)
    got = O.attention(qkv, w)
    for i in range(n):
        js = [j for j in range(n) if abs(i - j) <= w]
        s = np.array([qkv[i, :d] @ qkv[j, d:2 * d] / 8.0 for j in js], np.float64)
        p = np.exp(s - s.max())
        p /= p.sum()
        want = sum(pj * qkv[j, 2 * d:].astype(np.float64) for pj, j in zip(p, js))
        np.testing.assert_allclose(got[i], want, rtol=1e-5, atol=1e-6)
    qkv2 = qkv.copy()
    qkv2[8, d:] += 100.0  # key/value 8 is outside the window of query 5 (|5 - 8| = 3 > 2)
    assert np.allclose(O.attention(qkv2, w)[5], got[5])
    qkv2 = qkv.copy()
    qkv2[7, 2 * d:] += 100.0  # value 7 is inside (|5 - 7| = 2)
    assert not np.allclose(O.attention(qkv2, w)[5], got[5])


def test_geglu_against_torch():
    rng = np.random.default_rng(3)
    hh = rng.standard_normal((5, 64)).astype(np.float32) * 3
    want = (F.gelu(torch.from_numpy(hh[:, :32]).double()) * torch.from_numpy(hh[:, 32:]).double()).numpy()
    np.testing.assert_allclose(O.geglu(hh), want, rtol=1e-5, atol=2e-6)


def test_forward_against_the_golden_torch_restatement():
    g = np.load(os.path.join(GOLD, "forward_small.npz"))
    keys = ["d", "layers", "inter", "vocab", "head_layers", "head_ff", "n_qtypes", "window",
            "global_every", "max_positions", "norm_eps", "head_eps", "theta_global",
            "theta_local", "seed"]
    c = dict(zip(keys, g["cfg"].tolist()))
    c = {k: (float(v) if k in ("norm_eps", "head_eps", "theta_global", "theta_local") else int(v))
         for k, v in c.items()}
    m = O.Model(O.cfg(**c))
    for i in range(2):
        logits, trace, hx = m.forward(g[f"ids{i}"], int(g[f"qtype{i}"]), g[f"markers{i}"],
                                      trace=True, head_x=True)
        np.testing.assert_allclose(trace, g[f"trace{i}"], rtol=1e-4, atol=2e-5)
        np.testing.assert_allclose(hx, g[f"head{i}"], rtol=1e-4, atol=2e-5)
        np.testing.assert_allclose(logits, g[f"logits{i}"], rtol=1e-4, atol=2e-5)


def test_forward_against_torch_live():
    """The same restatement live, at the real Julia-1 width (d = 384, 6 heads) on a request
    longer than the window, with every third layer global."""
    c = dict(d=384, layers=4, inter=256, vocab=300, head_layers=2, head_ff=512, n_qtypes=3,
             window=64, global_every=3, max_positions=512, norm_eps=1e-5, head_eps=1e-5,
             theta_global=160000.0, theta_local=10000.0, seed=77)
    m = O.Model(O.cfg(**c))
    W = T.weights(lambda tid, cnt: O.synth(c["seed"], tid, cnt), c)
    rng = np.random.default_rng(4)
    ids = rng.integers(0, c["vocab"], 150)
    markers = np.array([0, 75, 149])
    torch.set_default_dtype(torch.float64)
    want, trace, _ = T.forward(W, c, torch.from_numpy(ids), 1, torch.from_numpy(markers))
    got, gt = m.forward(ids.astype(np.uint32), 1, markers.astype(np.uint32), trace=True)
    np.testing.assert_allclose(gt, torch.stack(trace).numpy(), rtol=1e-4, atol=5e-5)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-4, atol=5e-5)


# ---- the f16 emulation against the f32 oracle and the epilogue identities ------------------
def _ln_problem(rng, m, n, k, mean=0.0):
    x16 = rand16(rng, (m, k), mean=mean)
    W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    w16, cs = O.fold_layernorm(W, gamma)
    return x16, W, gamma, w16, cs


def test_emu_lnrope_is_layernorm_then_linear_then_rope():
    """The LayerNorm fold identity (src/prep.rs:6-13) and RoPE in the epilogue, through the
    emulation: rows with a large mean too (the cancellation the fold relies on)."""
    rng = np.random.default_rng(5)
    for mean in (0.0, 3.0):
        x16, W, gamma, w16, cs = _ln_problem(rng, 40, 384, 128, mean)
        table = O.rope_table(160000.0, 40)
        emu = O.emu_gemm(x16, w16, O.EPI_LN | O.EPI_ROPE, stats_in=O.row_stats(x16), colsum=cs,
                         rope=table, rope_cols=256)
        ref = O.rope_apply(O.linear(O.layernorm_rows(f32(x16), gamma, None, 1e-5), W), table)
        compare(f32(emu), ref, GEMM_REL if mean == 0 else 1e-2, what=f"emulated lnrope mean {mean}")


def test_emu_geglu_uses_the_interleave():
    rng = np.random.default_rng(6)
    inter = 128
    x16, W, gamma, w16, cs = _ln_problem(rng, 30, 2 * inter, 128)
    rows = O.geglu_rows(inter)
    emu = O.emu_gemm(x16, w16[rows], O.EPI_LN | O.EPI_GEGLU, stats_in=O.row_stats(x16),
                     colsum=cs[rows])
    ref = O.geglu(O.linear(O.layernorm_rows(f32(x16), gamma, None, 1e-5), W))
    compare(f32(emu), ref, GEMM_REL, what="emulated lngeglu")


def test_emu_resstats():
    rng = np.random.default_rng(7)
    a16, res16 = rand16(rng, (20, 192)), rand16(rng, (20, 128))
    w16 = rand16(rng, (128, 192), std=0.02)
    out, st = O.emu_gemm(a16, w16, O.EPI_RES | O.EPI_STATS, c16=res16)
    ref = f32(res16) + f32(a16).astype(np.float64) @ f32(w16).astype(np.float64).T
    compare(f32(out), ref, 1e-3, what="emulated resstats")
    check_stats(out, st)


def test_emu_attention_close_to_f64():
    rng = np.random.default_rng(8)
    qkv16 = rand16(rng, (100, 3 * 128))
    for w in (0, 8):
        compare(f32(O.emu_attention(qkv16, w)), O.attention(f32(qkv16), w), ATTN_REL,
                what=f"emulated attention w={w}")


# ---- tests of the tests -------------------------------------------------------------------
def _qkv_case():
    rng = np.random.default_rng(10)
    x16, W, gamma, w16, cs = _ln_problem(rng, 64, 384, 128)
    table = O.rope_table(160000.0, 64)
    emu = O.emu_gemm(x16, w16, O.EPI_LN | O.EPI_ROPE, stats_in=O.row_stats(x16), colsum=cs,
                     rope=table, rope_cols=256)
    ref = O.rope_apply(O.linear(O.layernorm_rows(f32(x16), gamma, None, 1e-5), W), table)
    return x16, W, gamma, w16, cs, table, emu, ref


def test_checks_reject_tiling_mistakes():
    """src/check.rs:860-871: a 64-column block left at zero and two swapped columns fail."""
    *_, emu, ref = _qkv_case()
    compare(f32(emu), ref, GEMM_REL)
    zeroed = emu.copy()
    zeroed[:, 64:128] = 0
    with pytest.raises(AssertionError):
        compare(f32(zeroed), ref, GEMM_REL)
    swapped = emu.copy()
    swapped[:, [3, 19]] = swapped[:, [19, 3]]
    with pytest.raises(AssertionError):
        compare(f32(swapped), ref, GEMM_REL)
    with pytest.raises(AssertionError):
        compare(f32(swapped), f32(emu), EMU_REL)


def test_checks_reject_a_missing_rope_or_a_wrong_pair():
    x16, W, gamma, w16, cs, table, emu, ref = _qkv_case()
    norope = O.emu_gemm(x16, w16, O.EPI_LN, stats_in=O.row_stats(x16), colsum=cs)
    with pytest.raises(AssertionError):
        compare(f32(norope), ref, 3e-2)
    # RoPE on adjacent pairs (2i, 2i + 1) instead of (i, i + 32): the reference's layout
    wrong = O.linear(O.layernorm_rows(f32(x16), gamma, None, 1e-5), W)
    for h in range(4):
        for i in range(32):
            c, s = table[:, i, 0], table[:, i, 1]
            a, b = wrong[:, 64 * h + 2 * i].copy(), wrong[:, 64 * h + 2 * i + 1].copy()
            wrong[:, 64 * h + 2 * i], wrong[:, 64 * h + 2 * i + 1] = a * c - b * s, b * c + a * s
    with pytest.raises(AssertionError):
        compare(wrong, ref, 3e-2)


def test_checks_reject_a_naive_geglu_order():
    rng = np.random.default_rng(11)
    inter = 128
    x16, W, gamma, w16, cs = _ln_problem(rng, 30, 2 * inter, 128)
    ref = O.geglu(O.linear(O.layernorm_rows(f32(x16), gamma, None, 1e-5), W))
    naive = O.emu_gemm(x16, w16, O.EPI_LN | O.EPI_GEGLU, stats_in=O.row_stats(x16), colsum=cs)
    with pytest.raises(AssertionError):
        compare(f32(naive), ref, 3e-2)


def test_checks_reject_a_missing_window_and_stats_errors():
    rng = np.random.default_rng(12)
    qkv16 = rand16(rng, (300, 3 * 128))
    ref = O.attention(f32(qkv16), 64)
    with pytest.raises(AssertionError):
        compare(f32(O.emu_attention(qkv16, 0)), ref, ATTN_REL)
    x16 = rand16(rng, (10, 128))
    st = O.row_stats(x16)
    check_stats(x16, st)
    bad = st.copy()
    bad[3, 1, 1] *= 1.01
    with pytest.raises(AssertionError):
        check_stats(x16, bad)


def test_checks_reject_a_two_ulp_embed_error():
    """src/check.rs:837-840: one value two f16 steps off fails the embed check (<= 1 ulp)."""
    rng = np.random.default_rng(13)
    table16 = rand16(rng, (50, 128))
    gamma = np.ones(128, np.float32)
    ids = np.arange(20, dtype=np.uint32)
    x = O.emu_embed(table16, gamma, ids)
    bad = x.copy()
    bad[5, 100] += 2
    assert O.ulps(x, x).max() == 0 and O.ulps(bad, x).max() == 2


def _np_layernorm64(x, gamma, eps):
    """LayerNorm of each row in float64 with numpy alone (no oracle code), weight gamma, no bias."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * np.asarray(gamma, np.float64)


def _f16_bits(x):
    return np.asarray(x, np.float64).astype(np.float16).view(np.uint16)


def test_emu_embed_is_the_layernorm_of_the_table_rows():
    """The f16 emulation of embed (oracle_emu_embed) against numpy's float64 LayerNorm of the
    gathered table rows, rounded once to f16: at most one f16 step apart (the emulation computes
    in f32), and a dropped gamma or a wrong row is caught."""
    rng = np.random.default_rng(21)
    d, vocab = 384, 200
    table16 = rand16(rng, (vocab, d), std=2.0, mean=0.3)
    gamma = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    ids = rng.integers(0, vocab, 64).astype(np.uint32)
    eps = 1e-5
    emu = O.emu_embed(table16, gamma, ids, eps)
    ref = _f16_bits(_np_layernorm64(f32(table16)[ids], gamma, eps))
    assert O.ulps(emu, ref).max() <= 1
    no_gamma = _f16_bits(_np_layernorm64(f32(table16)[ids], np.ones(d), eps))
    assert O.ulps(emu, no_gamma).max() > 1
    shifted = _f16_bits(_np_layernorm64(f32(table16)[(ids + 1) % vocab], gamma, eps))
    assert O.ulps(emu, shifted).max() > 1


def test_emu_norm_add_is_layernorm_plus_the_added_vector_with_stored_value_stats():
    """The f16 emulation of norm_add against numpy: float64 LayerNorm times gamma plus the added
    vector, rounded once to f16 (within one f16 step and 2^-10 relative), and its per-(row, 64-column) sums
    and sums of squares taken over the stored f16 values; a dropped add is caught."""
    rng = np.random.default_rng(22)
    n, d = 48, 768
    x16 = rand16(rng, (n, d), std=3.0, mean=0.5)
    gamma = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    add = (0.5 * rng.standard_normal(d)).astype(np.float32)
    eps = 1e-5
    out, st = O.emu_norm_add(x16, gamma, add, eps)
    ref64 = _np_layernorm64(f32(x16), gamma, eps) + add.astype(np.float64)
    ref = _f16_bits(ref64)
    # LN(x) . gamma + add cancels to small values in places, where the emulation's f32 rounding
    # moves a value by more than one of its tiny f16 steps: bound the value error instead there
    u = O.ulps(out, ref)
    assert (u > 1).mean() < 2e-3
    err = np.abs(out.view(np.float16).astype(np.float64) - ref64)
    assert np.all(err <= np.maximum(np.abs(ref64) * 2.0 ** -10, 1e-5))
    stored = out.view(np.float16).astype(np.float64).reshape(n, d // 64, 64)
    np.testing.assert_allclose(st[..., 0], stored.sum(axis=2), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(st[..., 1], (stored ** 2).sum(axis=2), rtol=1e-5, atol=1e-4)
    no_add = _f16_bits(_np_layernorm64(f32(x16), gamma, eps))
    assert O.ulps(out, no_add).max() > 1
