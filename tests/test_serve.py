"""The JSONL serve loop (the reference's src/serve.rs): answer() and the latency report's
percentiles on the CPU, pinned by closed forms; the julia-serve executable on the GPU, whose
results must carry exactly the logits julia_cuda_run gives for the same requests, the answer of
those logits, and the report on stderr.

answer() follows julia-rs's head::answer as the reference's own baseline tool writes its results
for tools/score.py to compare (tools/torch_baseline.py:214-226): softmax probabilities, the most
probable option for a choice, the expected option index for a score, p[1] for a noul. The
tokenizer and sequence() (julia-rs) are not part of this build: requests carry token ids, so the
tokenization of the reference's JSONL requests stays unpinned."""

import json
import math
import os
import re
import subprocess

import numpy as np
import pytest

import julia_hip as jh


def test_answer_closed_forms():
    # equal logits: uniform probabilities; the first of equal options is chosen
    v, p = jh.answer("choice", [0.25, 0.25, 0.25, 0.25])
    assert v == 0 and np.allclose(p, 0.25, rtol=0, atol=1e-15)
    # logits log 1, log 3: probabilities 1/4, 3/4
    v, p = jh.answer("choice", [0.0, math.log(3.0)])
    assert v == 1 and abs(p[0] - 0.25) < 1e-7 and abs(p[1] - 0.75) < 1e-7
    v, _ = jh.answer("noul", [0.0, math.log(3.0)])
    assert abs(v - 0.75) < 1e-7
    # score: the expected index; logits log(1), log(2), log(1) -> p = 1/4, 1/2, 1/4 -> 1
    v, p = jh.answer("score", [0.0, math.log(2.0), 0.0])
    assert abs(v - 1.0) < 1e-7 and abs(p.sum() - 1.0) < 1e-15
    # large logits do not overflow (shifted by the largest)
    v, p = jh.answer("choice", [1000.0, 1001.0, 999.0])
    e = np.exp(np.array([-1.0, 0.0, -2.0]))
    assert v == 1 and np.allclose(p, e / e.sum(), rtol=1e-12, atol=0)
    # one option
    v, p = jh.answer("score", [3.0])
    assert v == 0.0 and p[0] == 1.0


def test_answer_errors():
    with pytest.raises(jh.JuliaHipError, match="no options"):
        jh.answer("choice", [])
    with pytest.raises(jh.JuliaHipError, match="two options"):
        jh.answer("noul", [1.0])
    with pytest.raises(jh.JuliaHipError, match="nonfinite"):
        jh.answer("choice", [1.0, float("nan")])
    with pytest.raises(jh.JuliaHipError, match="question type"):
        jh.answer(3, [1.0, 2.0])


def test_latency_summary():
    """src/serve.rs:85: index round((n - 1) p) of the sorted values, halves away from zero."""
    vals = [5.0, 1.0, 4.0, 2.0, 3.0]
    assert jh.latency_summary(vals) == (3.0, 3.0, 5.0, 5.0, 5.0)
    # n = 2: p50 at index round(0.5) = 1 (Rust rounds half away from zero)
    assert jh.latency_summary([1.0, 2.0])[1] == 2.0
    # 101 values 0..100: p90 = 90, p99 = 99
    s = jh.latency_summary(np.arange(101.0)[::-1])
    assert s == (50.0, 50.0, 90.0, 99.0, 100.0)
    with pytest.raises(jh.JuliaHipError):
        jh.latency_summary([])


def test_serve_usage():
    assert os.path.exists(jh.SERVE_PATH), "julia-serve is not built"
    r = subprocess.run([jh.SERVE_PATH], capture_output=True, text=True, timeout=30)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([jh.SERVE_PATH, "synthetic", "--bogus"], capture_output=True, text=True,
                       timeout=30)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([jh.SERVE_PATH, "synthetic", "--max-length", "x"], capture_output=True,
                       text=True, timeout=30)
    assert r.returncode == 2 and "not a number" in r.stderr


def say(*a):
    print(*a, flush=True)


SMALL = "synthetic:d=384,layers=4,inter=1152,vocab=1000,head_ff=768,max_positions=2048,seed=7"


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [False, True])
def test_serve_results_match_julia_cuda_run(torch_cuda, tmp_path, fused):
    rng = np.random.default_rng(12)
    reqs = []
    for i in range(12):
        n = int(rng.integers(8, 400))
        k = int(rng.integers(2, 6))
        reqs.append((rng.integers(0, 1000, n).astype(np.uint32),
                     np.sort(rng.choice(n, k, replace=False)).astype(np.uint32), i % 3))
    lines = [json.dumps({"ids": r[0].tolist(), "markers": r[1].tolist(),
                         "type": jh.QTYPES[r[2]], "truncated": i == 5})
             for i, r in enumerate(reqs)]
    src = tmp_path / "requests.jsonl"
    src.write_text("\n".join(lines[:6]) + "\n\n" + "\n".join(lines[6:]) + "\n")
    cmd = [jh.SERVE_PATH, SMALL, "--max-length", "512"] + (["--layer-fused"] if fused else [])
    with open(src) as fh:
        r = subprocess.run(cmd, stdin=fh, capture_output=True, text=True, timeout=120)
    print(r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    out = [json.loads(x) for x in r.stdout.splitlines()]
    assert len(out) == len(reqs)
    # A child of this process, which holds the GPU's cooperative-launch resource, may have its
    # persistent launches refused: it then reports it and runs those requests per-step.
    refused = re.search(r"refused (\d+) cooperative launches", r.stderr)
    per_step = fused and refused is not None
    if per_step:
        say(f"julia-serve: {refused.group(1)} cooperative launches refused, compared per-step")
    with jh.Engine(SMALL, max_length=512) as e:
        want, _ = e.run(reqs, layer_fused=fused and not per_step)
    for i, (res, (ids, markers, q), w) in enumerate(zip(out, reqs, want)):
        np.testing.assert_array_equal(np.array(res["logits"], np.float32), w)
        v, p = jh.answer(q, w)
        np.testing.assert_allclose(res["probabilities"], p, rtol=1e-15, atol=0)
        assert res[jh.QTYPES[q]] == pytest.approx(v, rel=1e-15, abs=0)
        assert res["truncated"] == (i == 5)
    assert "per request, GPU (embed to logits)" in r.stderr
    assert f"{len(reqs)} requests" in r.stderr


@pytest.mark.gpu
def test_serve_rejects_untokenized_requests(torch_cuda, tmp_path):
    src = tmp_path / "r.jsonl"
    src.write_text(json.dumps({"ids": [1, 2, 3], "markers": [0, 2], "type": "choice"}) + "\n" +
                   json.dumps({"state": {}, "question": "q", "type": "choice",
                               "options": ["a", "b"]}) + "\n")
    with open(src) as fh:
        r = subprocess.run([jh.SERVE_PATH, SMALL], stdin=fh, capture_output=True, text=True,
                           timeout=120)
    assert r.returncode == 1 and "line 2" in r.stderr and "no tokenizer" in r.stderr
    assert len(r.stdout.splitlines()) == 1  # the first request was answered
