"""Independent float64 forwards of the three BASELINE training graphs, written
from the models' definitions ([3], [4]) and not from any
plan: no instruction words, no arena offsets, no kernel code.  Test
infrastructure: it pins the plan writer's lowering and the oracle's
instruction interpreter from outside (Step0Identity and central-difference
gradients, as the reference's system test does, test/system/
update_system_test.cc:78 and :208).

Definitions (the reference's operators, runtime/executor/*.cc, in exact
arithmetic):
- LoRA site: y = x W + s (x A) B with s = alpha / rank.
- LayerNorm: (x - mean) / sqrt(var + eps) * g + b, biased variance, eps 1e-5.
- RMSNorm: x / sqrt(mean(x^2) + eps) * g, eps 1e-5.
- GELU: the tanh form 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
- SiLU: x sigmoid(x).
- RoPE on each head's pairs (2c, 2c+1) at position p (the row's index within
  its sequence): angle p * base^(-2c/d), (a, b) -> (a cos - b sin,
  a sin + b cos).
- Causal attention per (sequence, head): softmax over j <= i of
  q_i . k_j / sqrt(d), heads interleaved along the row ([B*S, H*d]).
- Loss: mean over rows of -log softmax(logits)[label].
- int8 base: W = levels * column scale.
"""
from __future__ import annotations

import numpy as np

f64 = np.float64


def xent(logits, labels):
    z = logits - logits.max(axis=1, keepdims=True)
    lse = np.log(np.exp(z).sum(axis=1))
    return float(np.mean(lse - z[np.arange(len(labels)), labels]))


def layernorm(x, g, b, eps=1e-5):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def rmsnorm(x, g, eps=1e-5):
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * g


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def rope(x, B, S, H, d, base):
    pos = np.tile(np.arange(S, dtype=f64), B)[:, None]               # [T, 1]
    ang = pos * base ** (-2.0 * np.arange(d // 2, dtype=f64) / d)[None, :]
    c, s = np.cos(ang), np.sin(ang)                                  # [T, d/2]
    y = np.empty_like(x)
    for h in range(H):
        a, b = x[:, h * d:(h + 1) * d:2], x[:, h * d + 1:(h + 1) * d:2]
        y[:, h * d:(h + 1) * d:2] = a * c - b * s
        y[:, h * d + 1:(h + 1) * d:2] = a * s + b * c
    return y


def attention(q, k, v, B, S, H, d):
    out = np.empty_like(q)
    mask = np.triu(np.ones((S, S), bool), 1)
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        for h in range(H):
            cols = slice(h * d, (h + 1) * d)
            sc = q[rows, cols] @ k[rows, cols].T / np.sqrt(d)
            sc[mask] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[rows, cols] = p @ v[rows, cols]
    return out


def lora(x, W, A, Bm, s):
    return x @ W + s * ((x @ A) @ Bm)


def mlp_loss(P, x, labels, s):
    """din -> hidden (ReLU) -> dout, AddBias, LoRA on
    both MatMuls, softmax-xent."""
    x = np.asarray(x, f64)
    h = np.maximum(lora(x, P["W1"], P["A1"], P["B1"], s) + P["b1"], 0.0)
    return xent(lora(h, P["W2"], P["A2"], P["B2"], s) + P["b2"], labels)


def decoder_loss(P, tokens, labels, *, layers, heads, batch, seq, s, base=10000.0):
    """pre-norm blocks of LayerNorm, Q/K/V with LoRA on Q
    and V, RoPE on Q and K, causal attention, O, residual; LayerNorm, GELU
    FFN, residual; final LayerNorm, head, next-token xent."""
    x = P["emb"][tokens]
    D = x.shape[1]
    d = D // heads
    for l in range(layers):
        p = f"l{l}."
        n1 = layernorm(x, P[p + "g1"], P[p + "b1"])
        q = lora(n1, P[p + "wq"], P[p + "Aq"], P[p + "Bq"], s)
        k = n1 @ P[p + "wk"]
        v = lora(n1, P[p + "wv"], P[p + "Av"], P[p + "Bv"], s)
        q, k = rope(q, batch, seq, heads, d, base), rope(k, batch, seq, heads, d, base)
        x = x + attention(q, k, v, batch, seq, heads, d) @ P[p + "wo"]
        n2 = layernorm(x, P[p + "g2"], P[p + "b2"])
        x = x + gelu(n2 @ P[p + "wu"]) @ P[p + "wd"]
    return xent(layernorm(x, P["gf"], P["bf"]) @ P["wh"], labels)


def decoder_q8_loss(P, tokens, labels, *, layers, heads, batch, seq, s, base=10000.0):
    """pre-norm blocks of RMSNorm, Q/K/V/O on the int8
    base each with LoRA, RoPE, causal attention, residual; RMSNorm,
    SiLU-gated FFN on the int8 base, residual; final RMSNorm, f32 head."""
    x = P["emb"][tokens]
    D = x.shape[1]
    d = D // heads
    for l in range(layers):
        p = f"l{l}."
        n1 = rmsnorm(x, P[p + "g1"])
        q, k, v = (lora(n1, P[p + "w" + w], P[p + "A" + w], P[p + "B" + w], s) for w in "qkv")
        q, k = rope(q, batch, seq, heads, d, base), rope(k, batch, seq, heads, d, base)
        a = attention(q, k, v, batch, seq, heads, d)
        x = x + lora(a, P[p + "wo"], P[p + "Ao"], P[p + "Bo"], s)
        n2 = rmsnorm(x, P[p + "g2"])
        x = x + (silu(n2 @ P[p + "wg"]) * (n2 @ P[p + "wu"])) @ P[p + "wd"]
    return xent(rmsnorm(x, P["gf"]) @ P["wh"], labels)


def dequantized(arrays):
    """The model's weights in f64: int8 levels times their column scales."""
    out = {}
    for name, a in arrays.items():
        if name.endswith(".s"):
            continue
        if a.dtype == np.int8:
            out[name] = a.astype(f64) * arrays[name + ".s"].astype(f64)[None, :]
        else:
            out[name] = a.astype(f64)
    return out


def central_difference(loss, P, name, idx, h):
    """d loss / d P[name][idx] by (L(+h) - L(-h)) / 2h, in float64."""
    t = P[name]
    keep = t[idx]
    t[idx] = keep + h
    up = loss(P)
    t[idx] = keep - h
    down = loss(P)
    t[idx] = keep
    return (up - down) / (2 * h)
