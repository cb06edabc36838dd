"""Checkpoint directories for the tests: the seeded synthetic model written out as
model.safetensors + encoder/config.json, under the default tensor names of
julia-cuda_amd/csrc/checkpoint.h, so that loading it must give exactly the engine that the
"synthetic:..." spec of the same seed builds."""

import json
import os

import numpy as np

import julia_hip as jh
import oracle as O


def names(enc=""):
    """T_* tensor id -> default name (julia-cuda_amd/csrc/checkpoint.cpp's kNames)."""
    return {
        O.TOK_EMB: enc + "embeddings.tok_embeddings.weight",
        O.EMB_NORM: enc + "embeddings.norm.weight",
        O.FINAL_NORM: enc + "final_norm.weight",
        O.TYPE_EMB: "type_emb.weight",
    }


LAYER_NAMES = ["attn_norm.weight", "attn.Wqkv.weight", "attn.Wo.weight", "mlp_norm.weight",
               "mlp.Wi.weight", "mlp.Wo.weight"]
HEAD_NAMES = ["norm1.weight", "norm1.bias", "self_attn.in_proj_weight", "self_attn.in_proj_bias",
              "self_attn.out_proj.weight", "self_attn.out_proj.bias", "norm2.weight", "norm2.bias",
              "linear1.weight", "linear1.bias", "linear2.weight", "linear2.bias"]
SCORER_NAMES = ["norm.weight", "norm.bias", "lin1.weight", "lin1.bias", "lin2.weight", "lin2.bias"]


def tensors(c, seed, enc=""):
    """{name: (T_* id, shape)} of a model config c (d, layers, inter, vocab, head_layers,
    head_ff, n_qtypes)."""
    d, I, F = c["d"], c["inter"], c["head_ff"]
    out = {}
    nm = names(enc)
    out[nm[O.TOK_EMB]] = (O.TOK_EMB, (c["vocab"], d))
    out[nm[O.EMB_NORM]] = (O.EMB_NORM, (d,))
    out[nm[O.FINAL_NORM]] = (O.FINAL_NORM, (d,))
    out[nm[O.TYPE_EMB]] = (O.TYPE_EMB, (c.get("n_qtypes", 3), d))
    lshapes = [(d,), (3 * d, d), (d, d), (d,), (2 * I, d), (d, I)]
    for l in range(c["layers"]):
        for s, (n, shape) in enumerate(zip(LAYER_NAMES, lshapes)):
            if l == 0 and s == 0:
                continue  # ModernBERT's first layer has no attention LayerNorm
            out[f"{enc}layers.{l}.{n}"] = (O.LAYER_BASE + 16 * l + s, shape)
    hshapes = [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (F, d), (F,), (d, F), (d,)]
    for h in range(c["head_layers"]):
        for s, (n, shape) in enumerate(zip(HEAD_NAMES, hshapes)):
            out[f"head.layers.{h}.{n}"] = (O.HEAD_BASE + 32 * h + s, shape)
    sshapes = [(d,), (d,), (d, d), (d,), (1, d), (1,)]
    for s, (n, shape) in enumerate(zip(SCORER_NAMES, sshapes)):
        out[f"scorer.{n}"] = (O.SCORER_BASE + s, shape)
    return out


def write(path, c, seed, dtype=np.float32, enc="", config_extra=None, drop=(), reshape=None,
          gen=None):
    """Writes the synthetic model (seed) of config c as a checkpoint directory at path.
    gen(tid, shape, mean, std) -> f32 array: the tensors from another generator instead."""
    os.makedirs(os.path.join(path, "encoder"), exist_ok=True)
    arrays = {}
    for name, (tid, shape) in tensors(c, seed, enc).items():
        if name in drop:
            continue
        mean, std = O.dist(tid)
        if gen is None:
            v = jh.synth(seed, tid, int(np.prod(shape)), mean, std).reshape(shape)
        else:
            v = np.asarray(gen(tid, shape, mean, std), np.float32).reshape(shape)
        if reshape and name in reshape:
            v = v.reshape(reshape[name])
        if dtype == "bf16":  # round to nearest even into the top 16 bits
            u = v.astype(np.float32).view(np.uint32)
            u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
            arrays[name] = u.astype(np.uint16)
        else:
            arrays[name] = v.astype(dtype)
    save(os.path.join(path, "model.safetensors"), arrays, bf16=dtype == "bf16")
    cfg = {"hidden_size": c["d"], "num_hidden_layers": c["layers"], "intermediate_size": c["inter"],
           "vocab_size": c["vocab"], "max_position_embeddings": c.get("max_positions", 8192),
           "num_attention_heads": c["d"] // 64, "global_rope_theta": 160000.0,
           "local_rope_theta": 10000.0, "global_attn_every_n_layers": c.get("global_every", 3),
           "local_attention": 2 * c.get("window", 64), "norm_eps": 1e-5, "norm_bias": False,
           "hidden_activation": "gelu"}
    cfg.update(config_extra or {})
    with open(os.path.join(path, "encoder", "config.json"), "w") as fh:
        json.dump(cfg, fh)


def save(path, arrays, bf16=False, header_extra=None):
    """A safetensors file: u64 little-endian header length, the JSON header (name: dtype,
    shape, data_offsets into the data section), then the data. bf16: uint16 arrays are BF16."""
    kinds = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int32): "I32"}
    header, blobs, at = {}, [], 0
    for name, a in arrays.items():
        a = np.ascontiguousarray(a)
        kind = "BF16" if (bf16 and a.dtype == np.uint16) else kinds[a.dtype]
        raw = a.tobytes()
        header[name] = {"dtype": kind, "shape": list(a.shape), "data_offsets": [at, at + len(raw)]}
        blobs.append(raw)
        at += len(raw)
    header["__metadata__"] = {"format": "pt"}
    header.update(header_extra or {})
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as fh:
        fh.write(len(text).to_bytes(8, "little") + text)
        for raw in blobs:
            fh.write(raw)
