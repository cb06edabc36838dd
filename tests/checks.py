"""Parity checks and their limits, shared by the tests.

Limits: the north star's (an output's max |error| over max |reference| <= 2e-2 in f16 storage,
final logits mean |diff| <= 0.03 and max |diff| <= 0.1, row statistics within 1e-3 relative)
and the reference's own per-step limits against its f32 reference (src/check.rs:382-389: GEMM
outputs 2e-3 and attention 4e-3 Frobenius-relative; against the f16 emulation of the kernel's
arithmetic 1e-3, src/check.rs:156)."""

import numpy as np

import oracle as O

MAX_REL = 2e-2      # max |a - b| / max |b|
GEMM_REL = 2e-3     # ||a - b|| / ||b|| vs the f32 reference
ATTN_REL = 4e-3
EMU_REL = 1e-3      # vs the f16 emulation
STATS_REL = 1e-3
LOGIT_MEAN = 0.03
LOGIT_MAX = 0.1


def f32(x16):
    return O.f16_bits_to_f32(x16)


def compare(got, ref, rel_limit, max_limit=MAX_REL, what="output"):
    """Frobenius and element-wise (max over max) relative error of got against ref; raises on a
    miss, returns (rel, maxrel)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    rel, mrel = O.rel_err(got, ref), O.max_rel(got, ref)
    assert rel <= rel_limit and mrel <= max_limit, (
        f"{what}: relative error {rel:.3e} (limit {rel_limit:.1e}), max {mrel:.3e} "
        f"(limit {max_limit:.1e})")
    return rel, mrel


def stats_err(x16, stats):
    """src/check.rs:281-293 `stats_err`: the largest |dS| / sqrt(Q) and |dQ| / Q over the rows,
    against f64 sums of the stored f16 row; stats is [rows][groups][2] (summed over groups)."""
    x = f32(x16).astype(np.float64)
    s_ref = x.sum(axis=1)
    q_ref = np.maximum((x * x).sum(axis=1), 1e-30)
    st = np.asarray(stats, np.float64).reshape(x.shape[0], -1, 2)
    s, q = st[:, :, 0].sum(axis=1), st[:, :, 1].sum(axis=1)
    return float(max(np.max(np.abs(s - s_ref) / np.sqrt(q_ref)), np.max(np.abs(q - q_ref) / q_ref)))


def check_stats(x16, stats, what="stats"):
    e = stats_err(x16, stats)
    assert e <= STATS_REL, f"{what}: row statistics {e:.3e} off (limit {STATS_REL:.0e})"
    return e


def check_logits(got, ref, what="logits"):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got)), what
    d = np.abs(got - ref)
    assert d.mean() <= LOGIT_MEAN and d.max() <= LOGIT_MAX, (
        f"{what}: mean |diff| {d.mean():.4f} (limit {LOGIT_MEAN}), max {d.max():.4f} "
        f"(limit {LOGIT_MAX})")
    return float(d.mean()), float(d.max())


def rand16(rng, shape, std=1.0, mean=0.0):
    return O.to_f16_bits(rng.standard_normal(shape).astype(np.float32) * std + mean)
