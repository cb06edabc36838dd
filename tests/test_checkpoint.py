"""Checkpoint directories (the reference's src/checkpoint.rs:27-62 + src/weights.rs:143-238):
the config and tensor checks on the CPU, and on the GPU that a checkpoint holding the seeded
synthetic model's tensors gives exactly the engine the "synthetic:..." spec of the same seed
builds (the same preparation from either source), in F32, and within the logit tolerance in
BF16; both against the f32 oracle; and a checkpoint of weights from an independent generator
against the torch restatement of the forward pass, which reads the tensors in the public
conventions (torch Linear weights [out][in], ModernBERT's Wqkv rows q | k | v and Wi rows
input | gate), so a transposed matrix or a swapped split fails.

The tensor names are an assumption (julia-rs, which holds the reference's checkpoint reader, is
not vendored, and no real Julia-1 checkpoint is available): parity with a real checkpoint's
names stays unpinned."""

import json
import os
import sys

import numpy as np
import pytest

import ckpt
import julia_hip as jh
import oracle as O
from checks import check_logits

TINY = dict(d=128, layers=2, inter=256, vocab=100, head_layers=1, head_ff=256, n_qtypes=3,
            window=32, global_every=2, max_positions=512)


def test_config_from_a_checkpoint(tmp_path):
    ckpt.write(str(tmp_path), TINY, seed=3)
    i = jh.checkpoint_config(str(tmp_path))
    got = {k: getattr(i, k) for k in ("d", "layers", "inter", "vocab", "head_layers", "head_ff",
                                       "n_qtypes", "window", "global_every", "max_positions")}
    assert got == TINY
    assert abs(i.norm_eps - 1e-5) < 1e-9 and abs(i.head_eps - 1e-5) < 1e-9


def test_encoder_prefix_dtypes_and_julia_config(tmp_path):
    """The encoder's key prefix is found from the embedding table's name; F16 and BF16 tensors
    are read; julia_config.json sets the head's LayerNorm eps."""
    for k, dt in enumerate((np.float16, "bf16")):
        d = str(tmp_path / f"m{k}")
        ckpt.write(d, TINY, seed=3, dtype=dt, enc="model.")
        with open(os.path.join(d, "julia_config.json"), "w") as fh:
            json.dump({"head_norm_eps": 1e-6}, fh)
        i = jh.checkpoint_config(d)
        assert i.layers == 2 and abs(i.head_eps - 1e-6) < 1e-12


def test_tensor_name_overrides(tmp_path):
    """julia_hip_names.json renames tensors (patterns with {enc}, {l}, {h})."""
    d = str(tmp_path)
    ckpt.write(d, TINY, seed=3)
    path = os.path.join(d, "model.safetensors")
    blob = open(path, "rb").read()
    n = int.from_bytes(blob[:8], "little")
    header = json.loads(blob[8:8 + n])
    renamed = {k.replace("head.layers.", "julia.head.").replace("self_attn.", "attn.") if
               k.startswith("head.") else k: v for k, v in header.items()}
    text = json.dumps(renamed).encode()
    text += b" " * (-len(text) % 8)
    open(path, "wb").write(len(text).to_bytes(8, "little") + text + blob[8 + n:])
    # without the overrides no head layer is found (the count is read off the tensors)
    assert jh.checkpoint_config(d).head_layers == 0
    over = {f"head.{k}": f"julia.head.{{h}}.{v.replace('self_attn.', 'attn.')}"
            for k, v in zip(["norm1_w", "norm1_b", "in_proj_w", "in_proj_b", "out_proj_w",
                             "out_proj_b", "norm2_w", "norm2_b", "linear1_w", "linear1_b",
                             "linear2_w", "linear2_b"], ckpt.HEAD_NAMES)}
    with open(os.path.join(d, "julia_hip_names.json"), "w") as fh:
        json.dump(over, fh)
    assert jh.checkpoint_config(d).head_layers == 1
    with open(os.path.join(d, "julia_hip_names.json"), "w") as fh:
        json.dump({"head.bogus": "x"}, fh)
    with pytest.raises(jh.JuliaHipError, match="unknown tensor 'head.bogus'"):
        jh.checkpoint_config(d)


@pytest.mark.parametrize("case", ["missing", "shape", "dtype", "truncated", "no_config",
                                  "heads", "norm_bias", "header"])
def test_checkpoint_errors(tmp_path, case):
    d = str(tmp_path)
    if case == "missing":
        ckpt.write(d, TINY, seed=3, drop=("layers.1.attn.Wo.weight",))
        match = "no tensor 'layers.1.attn.Wo.weight'"
    elif case == "shape":
        ckpt.write(d, TINY, seed=3, reshape={"layers.1.mlp.Wi.weight": (256, 256)})
        match = r"'layers.1.mlp.Wi.weight' is \[256, 256\], the config says \[512, 128\]"
    elif case == "dtype":
        ckpt.write(d, TINY, seed=3)
        arrays = {"final_norm.weight": np.ones(128, np.int32)}
        _merge(d, arrays)
        match = "F32, F16 or BF16 only"
    elif case == "truncated":
        ckpt.write(d, TINY, seed=3)
        p = os.path.join(d, "model.safetensors")
        blob = open(p, "rb").read()
        open(p, "wb").write(blob[:len(blob) - 1000])
        match = "lies outside the file"
    elif case == "no_config":
        ckpt.write(d, TINY, seed=3)
        os.remove(os.path.join(d, "encoder", "config.json"))
        match = "no model at"
    elif case == "heads":
        ckpt.write(d, TINY, seed=3, config_extra={"num_attention_heads": 4})
        match = "heads of 64 only"
    elif case == "norm_bias":
        ckpt.write(d, TINY, seed=3, config_extra={"norm_bias": True})
        match = "norm_bias"
    else:
        ckpt.write(d, TINY, seed=3)
        p = os.path.join(d, "model.safetensors")
        blob = open(p, "rb").read()
        open(p, "wb").write((len(blob) * 2).to_bytes(8, "little") + blob[8:])
        match = "header length"
    with pytest.raises(jh.JuliaHipError, match=match):
        jh.checkpoint_config(d)
    # julia_cuda_load checks the directory the same way before it looks for a GPU
    with pytest.raises(jh.JuliaHipError, match=match):
        jh.Engine(d)


def _merge(d, extra):
    """Replaces tensors of a checkpoint (same names) with `extra`."""
    p = os.path.join(d, "model.safetensors")
    blob = open(p, "rb").read()
    n = int.from_bytes(blob[:8], "little")
    header = json.loads(blob[8:8 + n])
    data = blob[8 + n:]
    arrays = {}
    kinds = {"F32": np.float32, "F16": np.float16, "I32": np.int32}
    for k, v in header.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        arrays[k] = np.frombuffer(data[a:b], kinds[v["dtype"]]).reshape(v["shape"])
    arrays.update(extra)
    ckpt.save(p, arrays)


# ---- GPU: the same engine from either source ----------------------------------------------------
SMALL = dict(d=384, layers=4, inter=1152, vocab=1000, head_layers=2, head_ff=768, n_qtypes=3,
             window=64, global_every=3, max_positions=2048)
SEED = 7


def _spec():
    keys = ("d", "layers", "inter", "vocab", "head_layers", "head_ff", "window", "global_every",
            "max_positions")
    return "synthetic:" + ",".join(f"{k}={SMALL[k]}" for k in keys) + f",seed={SEED}"


def _requests(rng):
    out = []
    for n in (72, 293, 400):
        ids = rng.integers(0, SMALL["vocab"], n).astype(np.uint32)
        out.append((ids, [1, n // 2, n - 1], int(rng.integers(0, 3))))
    return out


@pytest.mark.gpu
def test_checkpoint_engine_matches_the_synthetic_engine(torch_cuda, tmp_path):
    d = str(tmp_path / "f32")
    ckpt.write(d, SMALL, seed=SEED, enc="model.")
    rng = np.random.default_rng(5)
    reqs = _requests(rng)
    a = jh.Engine(_spec(), max_length=512)
    b = jh.Engine(d, max_length=512)
    for name, idx in (("tok_emb", 0), ("wqkv", 1), ("wi", 2), ("in_proj", 1), ("lin1", 0)):
        assert np.array_equal(a.tensor_host(name, idx), b.tensor_host(name, idx)), name
    for fused in (False, True):
        la, _ = a.run(reqs, layer_fused=fused)
        lb, _ = b.run(reqs, layer_fused=fused)
        for x, y in zip(la, lb):
            assert np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32))
    a.close()
    b.close()


@pytest.mark.gpu
def test_bf16_checkpoint_within_the_logit_tolerance(torch_cuda, tmp_path):
    d32, d16 = str(tmp_path / "f32"), str(tmp_path / "bf16")
    ckpt.write(d32, SMALL, seed=SEED)
    ckpt.write(d16, SMALL, seed=SEED, dtype="bf16")
    reqs = _requests(np.random.default_rng(6))
    a = jh.Engine(d32, max_length=512)
    b = jh.Engine(d16, max_length=512)
    la, _ = a.run(reqs)
    lb, _ = b.run(reqs)
    x, y = np.concatenate([np.asarray(v) for v in la]), np.concatenate([np.asarray(v) for v in lb])
    assert np.isfinite(y).all()
    assert np.abs(x - y).mean() <= 0.03 and np.abs(x - y).max() <= 0.1, (x, y)
    a.close()
    b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [np.float32, "bf16"])
def test_checkpoint_engine_matches_the_oracle(torch_cuda, tmp_path, dtype):
    """src/checkpoint.rs:27-62 + src/weights.rs:257-271: the engine loaded from a checkpoint
    directory (F32, and BF16 rounded) against the f32 oracle's forward pass of the same seeded
    model, per-step kernels and the whole-model launch."""
    d = str(tmp_path / "ck")
    ckpt.write(d, SMALL, seed=SEED, dtype=dtype, enc="model.")
    keys = ("d", "layers", "inter", "vocab", "head_layers", "head_ff", "window", "global_every",
            "max_positions")
    m = O.Model(O.cfg(**{k: SMALL[k] for k in keys}, seed=SEED))
    reqs = _requests(np.random.default_rng(8))
    e = jh.Engine(d, max_length=512)
    try:
        for fused in (False, True):
            out, _ = e.run(reqs, layer_fused=fused)
            for (ids, markers, q), lg in zip(reqs, out):
                mean, mx = check_logits(lg, m.forward(ids, q, markers),
                                        f"{dtype} checkpoint, fused={fused}, {len(ids)} tokens")
                print(f"{dtype} fused={fused} n={len(ids)}: mean |d| {mean:.2e} max {mx:.2e}",
                      flush=True)
    finally:
        e.close()


@pytest.mark.gpu
def test_independent_checkpoint_matches_the_torch_restatement(torch_cuda, tmp_path):
    """Weights from numpy's generator (not the synthetic stream the engine and the oracle share),
    written under the checkpoint's names, against tests/golden/torch_reference.py's forward pass
    on the same tensors read as torch Linear weights ([out][in]), Wqkv as q | k | v rows and Wi
    as input | gate rows (GELU(input) * gate): this pins the loader's orientation and split
    orders independently of the synthetic model."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import torch

    import torch_reference as T

    rng = np.random.default_rng(2024)
    store = {}

    def gen(tid, shape, mean, std):
        a = (mean + std * rng.standard_normal(shape)).astype(np.float32)
        store[tid] = a
        return a

    d = str(tmp_path / "indep")
    ckpt.write(d, SMALL, seed=0, gen=gen, enc="model.")
    cfg = dict(SMALL, norm_eps=1e-5, head_eps=1e-5, theta_global=160000.0, theta_local=10000.0)

    def synth(tid, count):  # layer 0's attention LayerNorm is not in the checkpoint (unused)
        a = store.get(tid)
        return np.zeros(count, np.float32) if a is None else a.reshape(-1)[:count]

    W = T.weights(synth, cfg)
    reqs = _requests(np.random.default_rng(9))
    e = jh.Engine(d, max_length=512)
    try:
        for fused in (False, True):
            out, _ = e.run(reqs, layer_fused=fused)
            for (ids, markers, q), lg in zip(reqs, out):
                want, _, _ = T.forward(W, cfg, torch.from_numpy(ids.astype(np.int64)), q,
                                       torch.tensor(markers, dtype=torch.int64))
                mean, mx = check_logits(lg, want.numpy(), f"fused={fused}, {len(ids)} tokens")
                print(f"independent fused={fused} n={len(ids)}: mean |d| {mean:.2e} "
                      f"max {mx:.2e}", flush=True)
    finally:
        e.close()
