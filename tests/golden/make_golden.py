"""Writes tests/golden/*.npz: the fixtures that pin the oracle.

    python tests/golden/make_golden.py

forward_small.npz: a small Julia-1-shaped model (the synthetic generator's weights) run by the
independent torch f64 restatement in torch_reference.py on two requests: the logits, the
residual stream after each encoder layer and the head's stream. test_oracle.py checks the C
oracle's forward pass against it.

ops.npz: textbook ops from library routines on seeded inputs: LayerNorm (torch), attention
(torch scaled_dot_product_attention, global and +-3 window), erf-GELU (math.erf), RoPE (complex
rotation).
"""

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402
import torch_reference as T  # noqa: E402

SMALL = dict(d=128, layers=4, inter=128, vocab=500, head_layers=2, head_ff=256, n_qtypes=3,
             window=4, global_every=3, max_positions=256, norm_eps=1e-5, head_eps=1e-5,
             theta_global=160000.0, theta_local=10000.0, seed=1234)


def forward_small():
    c = SMALL
    W = T.weights(lambda tid, cnt: O.synth(c["seed"], tid, cnt), c)
    out = {}
    rng = np.random.default_rng(5)
    for i, (n, q) in enumerate([(20, 0), (37, 2)]):
        ids = rng.integers(0, c["vocab"], n)
        markers = np.sort(rng.choice(n, 3, replace=False))
        logits, trace, hx = T.forward(W, c, torch.from_numpy(ids), q, torch.from_numpy(markers))
        out[f"ids{i}"] = ids.astype(np.uint32)
        out[f"markers{i}"] = markers.astype(np.uint32)
        out[f"qtype{i}"] = np.array(q)
        out[f"logits{i}"] = logits.numpy()
        out[f"trace{i}"] = torch.stack(trace).numpy()
        out[f"head{i}"] = hx.numpy()
    out["cfg"] = np.array(list(c.values()), dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "forward_small.npz"), **out)


def ops():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 192)) * 2 + 0.5
    g, b = 1 + 0.1 * rng.standard_normal(192), 0.1 * rng.standard_normal(192)
    ln = torch.nn.functional.layer_norm(torch.from_numpy(x), (192,), torch.from_numpy(g),
                                        torch.from_numpy(b), 1e-5).numpy()
    qkv = rng.standard_normal((11, 3 * 128))
    q, k, v = (torch.from_numpy(qkv[:, i * 128:(i + 1) * 128]) for i in range(3))
    att_g = T.attention(q, k, v, 2, 0).numpy()
    att_w = T.attention(q, k, v, 2, 3).numpy()
    xs = np.linspace(-8, 8, 161)
    gelu = np.array([v * 0.5 * (1 + math.erf(v / math.sqrt(2))) for v in xs])
    rq = rng.standard_normal((5, 128))
    rope = T.rope(torch.from_numpy(rq), 10000.0, 2).numpy()
    np.savez_compressed(os.path.join(HERE, "ops.npz"), ln_x=x, ln_g=g, ln_b=b, ln=ln, qkv=qkv,
                        att_global=att_g, att_window3=att_w, gelu_x=xs, gelu=gelu, rope_x=rq,
                        rope=rope)


if __name__ == "__main__":
    torch.set_default_dtype(torch.float64)
    forward_small()
    ops()
    print("wrote", os.listdir(HERE))
