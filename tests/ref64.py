"""Float64 numpy statements of the hot-path mathematics, used only to pin the
CPU oracle (and through it the GPU path) on small shapes. Written from the
published formulas (GELU, LayerNorm, softmax attention, GPT-2, DistilBERT), not
from the oracle's code: different language, precision and summation order,
so a dropped term, a wrong sign, index or transpose shows up as a mismatch.
"""
from __future__ import annotations

import math

import numpy as np


def gelu_erf(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))


def gelu_tanh(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def layernorm(x, g, b, eps):
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def softmax(x, axis=-1):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis, keepdims=True))
    return e / e.sum(axis, keepdims=True)


def attention(q, k, v, head_dim, mask=None, fill=-1e30, causal=False):
    """q,k,v [B,S,H]; mask broadcastable to [B,nH,S,S], True = masked."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    B, S, H = q.shape
    nH = H // head_dim
    qh = q.reshape(B, S, nH, head_dim).transpose(0, 2, 1, 3)
    kh = k.reshape(B, S, nH, head_dim).transpose(0, 2, 1, 3)
    vh = v.reshape(B, S, nH, head_dim).transpose(0, 2, 1, 3)
    s = qh @ kh.transpose(0, 1, 3, 2) / math.sqrt(head_dim)
    if mask is not None:
        s = np.where(np.broadcast_to(np.asarray(mask, bool), s.shape), fill, s)
    if causal:
        s = np.where(np.triu(np.ones((S, S), bool), 1), fill, s)
    o = softmax(s) @ vh
    return o.transpose(0, 2, 1, 3).reshape(B, S, H)


def encoder(cfg, w, ids, mask):
    """DistilBERT-style post-LN encoder + classifier head, weights in the
    order of inferc_amd.graphs.encoder_weights."""
    H, L = cfg["hidden"], cfg["layers"]
    hd = H // cfg["heads"]
    w = [np.asarray(t, np.float64) for t in w]
    B, S = ids.shape
    h = layernorm(w[0][ids] + w[1][np.arange(S)][None], w[2], w[3], cfg["eps"])
    m = (np.asarray(mask) == 0)[:, None, None, :]
    for l in range(L):
        p = w[4 + 16 * l: 4 + 16 * (l + 1)]
        q, k, v = h @ p[0] + p[1], h @ p[2] + p[3], h @ p[4] + p[5]
        ctx = attention(q, k, v, hd, m, fill=float(np.finfo(np.float32).min))
        h = layernorm(ctx @ p[6] + p[7] + h, p[8], p[9], cfg["eps"])
        f = gelu_erf(h @ p[10] + p[11])
        h = layernorm(f @ p[12] + p[13] + h, p[14], p[15], cfg["eps"])
    t = w[4 + 16 * L:]
    pre = np.maximum(h[:, 0] @ t[0].T + t[1], 0.0)
    return pre @ t[2].T + t[3]


def gpt2_logits(cfg, w, ids):
    """Full-sequence GPT-2 (pre-LN, causal, tied head) logits [n, V]."""
    H, L = cfg["hidden"], cfg["layers"]
    hd = H // cfg["heads"]
    w = [np.asarray(t, np.float64) for t in w]
    n = len(ids)
    h = w[0][ids] + w[1][np.arange(n)]
    for l in range(L):
        p = w[2 + 12 * l: 2 + 12 * (l + 1)]
        a = layernorm(h, p[0], p[1], cfg["eps"])
        qkv = a @ p[2] + p[3]
        q, k, v = qkv[:, :H], qkv[:, H:2 * H], qkv[:, 2 * H:]
        att = attention(q[None], k[None], v[None], hd, causal=True,
                        fill=float(np.finfo(np.float32).min))[0]
        h = h + (att @ p[4] + p[5])
        a = layernorm(h, p[6], p[7], cfg["eps"])
        h = h + (gelu_tanh(a @ p[8] + p[9]) @ p[10] + p[11])
    hf = layernorm(h, w[2 + 12 * L], w[3 + 12 * L], cfg["eps"])
    return hf @ w[0].T


def int4_deq(W, scales, K):
    """s_r * float(nib - 8) as float32 products."""
    W = np.asarray(W, np.uint8)
    nib = np.empty((W.shape[0], K), np.int64)
    nib[:, 0::2] = W & 0xF
    nib[:, 1::2] = W >> 4
    return (np.asarray(scales, np.float32)[:, None] * (nib - 8).astype(np.float32)).astype(
        np.float32)
