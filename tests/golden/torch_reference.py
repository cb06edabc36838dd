"""An independent restatement of the Julia-1-shaped forward pass in torch (f64, CPU), built from
library routines: torch.nn.functional.layer_norm, linear, scaled_dot_product_attention (with an
explicit boolean band mask for the sliding window), the exact erf GELU, and RoPE as a complex
rotation. It shares no code with the C oracle; tests/test_oracle.py and the committed golden
fixtures (make_golden.py) use it to pin the oracle's forward pass.

The model (what the reference's src/check.rs `trace` :177-224 and `head_trace` :484-548 compute
with julia-rs): embed + LayerNorm (no bias); per layer, LN (absent in layer 0) -> Wqkv -> RoPE on
q and k (theta_global in every `global_every`-th layer, else theta_local, with attention limited
to |i - j| <= window) -> attention -> Wo + residual -> LN -> Wi -> GeGLU -> Wo_mlp + residual;
then the final LN + type embedding, pre-LN head layers (LN with bias, in_proj + bias, global
attention without RoPE, out_proj + bias + residual, LN, linear1 + bias, ReLU, linear2 + bias +
residual), and the scorer on the marker rows (LN, lin1 + bias, GELU, lin2 + bias).
"""

import math

import torch
import torch.nn.functional as F


def rope(x, theta, heads):
    """Rotate-half RoPE on [n, heads*64]: dims (i, i + 32) of each head as the complex number
    x_i + j x_{i+32}, multiplied by exp(j p theta^(-2i/64))."""
    n = x.shape[0]
    x = x.view(n, heads, 2, 32)
    z = torch.complex(x[:, :, 0, :], x[:, :, 1, :])
    inv = theta ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64.0)
    ang = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
    z = z * torch.polar(torch.ones_like(ang), ang)[:, None, :]
    return torch.stack([z.real, z.imag], dim=2).reshape(n, heads * 64)


def attention(q, k, v, heads, window):
    n = q.shape[0]
    sh = lambda t: t.view(n, heads, 64).transpose(0, 1)
    mask = None
    if window > 0:
        i = torch.arange(n)
        mask = (i[:, None] - i[None, :]).abs() <= window
    o = F.scaled_dot_product_attention(sh(q), sh(k), sh(v), attn_mask=mask)
    return o.transpose(0, 1).reshape(n, heads * 64)


def gelu(x):
    return F.gelu(x, approximate="none")


def forward(W, cfg, ids, qtype, markers):
    """W: dict of f64 tensors named as in the oracle (see weights()); returns (logits, [x after
    each encoder layer], head stream)."""
    d = cfg["d"]
    heads = d // 64
    eps, heps = cfg["norm_eps"], cfg["head_eps"]
    ln = lambda x, g, b=None, e=eps: F.layer_norm(x, (d,), g, b, e)
    x = ln(W["tok_emb"][ids], W["emb_norm"])
    trace = []
    for l in range(cfg["layers"]):
        P = W["layers"][l]
        glob = l % cfg["global_every"] == 0
        h = x if l == 0 else ln(x, P["attn_norm"])
        qkv = F.linear(h, P["wqkv"])
        th = cfg["theta_global"] if glob else cfg["theta_local"]
        q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
        q, k = rope(q, th, heads), rope(k, th, heads)
        x = x + F.linear(attention(q, k, v, heads, 0 if glob else cfg["window"]), P["wo"])
        hh = F.linear(ln(x, P["mlp_norm"]), P["wi"])
        inter = hh.shape[1] // 2
        x = x + F.linear(gelu(hh[:, :inter]) * hh[:, inter:], P["wo_mlp"])
        trace.append(x.clone())
    x = ln(x, W["final_norm"]) + W["type_emb"][qtype]
    for P in W["head"]:
        h = ln(x, P["norm1_w"], P["norm1_b"], heps)
        qkv = F.linear(h, P["in_proj_w"], P["in_proj_b"])
        a = attention(qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:], heads, 0)
        x = x + F.linear(a, P["out_proj_w"], P["out_proj_b"])
        h = ln(x, P["norm2_w"], P["norm2_b"], heps)
        x = x + F.linear(F.relu(F.linear(h, P["linear1_w"], P["linear1_b"])), P["linear2_w"],
                         P["linear2_b"])
    S = W["scorer"]
    z = ln(x[markers], S["norm_w"], S["norm_b"], heps)
    y = gelu(F.linear(z, S["lin1_w"], S["lin1_b"]))
    logits = F.linear(y, S["lin2_w"], S["lin2_b"])[:, 0]
    return logits, trace, x


def weights(synth, cfg):
    """The synthetic model's raw (unfolded) weights from `synth(tid, count) -> float32 array`
    (the oracle's generator), as f64 tensors."""
    d, I, FF = cfg["d"], cfg["inter"], cfg["head_ff"]
    t = lambda tid, *shape: torch.from_numpy(synth(tid, math.prod(shape)).reshape(shape)).double()
    W = {"emb_norm": t(2, d), "final_norm": t(3, d), "type_emb": t(4, cfg["n_qtypes"], d),
         "layers": [], "head": []}
    for l in range(cfg["layers"]):
        b = 100 + 16 * l
        W["layers"].append({"attn_norm": t(b + 0, d), "wqkv": t(b + 1, 3 * d, d), "wo": t(b + 2, d, d),
                            "mlp_norm": t(b + 3, d), "wi": t(b + 4, 2 * I, d),
                            "wo_mlp": t(b + 5, d, I)})
    names = ["norm1_w", "norm1_b", "in_proj_w", "in_proj_b", "out_proj_w", "out_proj_b",
             "norm2_w", "norm2_b", "linear1_w", "linear1_b", "linear2_w", "linear2_b"]
    shapes = [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (FF, d), (FF,), (d, FF),
              (d,)]
    for h in range(cfg["head_layers"]):
        W["head"].append({nm: t(1000 + 32 * h + i, *sh) for i, (nm, sh) in enumerate(zip(names, shapes))})
    snames = ["norm_w", "norm_b", "lin1_w", "lin1_b", "lin2_w", "lin2_b"]
    sshapes = [(d,), (d,), (d, d), (d,), (1, d), (1,)]
    W["scorer"] = {nm: t(2000 + i, *sh) for i, (nm, sh) in enumerate(zip(snames, sshapes))}
    W["tok_emb"] = t(1, cfg["vocab"], d)
    return W
