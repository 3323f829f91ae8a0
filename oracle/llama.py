"""CPU restatement of the reference's Llama forward -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``__graft_entry__.smoke()`` may import this module, and
only as the checker of the device decode runner (rq_llama_*), never as the
product path.

It computes, in float64, the logits of every position of a token sequence
under causal attention -- the whole sequence at once, so it shares no code
path with the device's one-position-at-a-time KV-cache loop.  Inputs are the
same host weights the device gets: fp16 embeddings and norm weights, per-row
int8 codes with f32 scales (dequantized exactly, W = q * s) or affine u8
codes with f32 group scales and biases (W = u * s + b, exact in f64).  No
intermediate rounding: the reference computes in f32 throughout; the device rounds
activations entering a GEMV and the KV cache to fp16, and its tests state the
tolerance that allows for that.

Reference semantics followed (file:line):
  rmsnorm   rusty-backend/src/kernels.wgsl:87-102   x * (1/sqrt(mean(x^2) + eps)) * w,
            applied to every row (the reference kernel stops after row 0:
            `if (row >= 1u) { return; }`, :91 -- a defect not restated)
  rope      kernels.wgsl:60-79    rotate-half pairs (d, d + hd/2), angle
            pos * theta^(-2d/hd); here each token uses its own position
            (the reference passes one `pos` per call, rusty-graph/src/lib.rs:204-205)
  attention rusty-graph/src/lib.rs:191-283 + flash_attention_v2.wgsl:79-83:
            GQA head h reads KV head h // (n_heads / n_kv), scale 1/sqrt(hd),
            causal softmax
  silu      kernels.wgsl:104-113  v / (1 + exp(-v)); MLP lib.rs:317-323
  block     lib.rs:364-378        x + attn(norm1(x)); h + mlp(norm2(h))
  model     lib.rs:420-436        embed -> blocks -> norm -> lm_head
  greedy    kernels.wgsl:173-188  first index of the largest value > -1e9

Pinning (tests/test_oracle_llama.py): rmsnorm closed forms and scale
invariance; rope identity at position 0, pair-norm preservation and the
relative-position property of rotated dot products; attention against a
single key and against equal keys; the GQA index via duplicated-KV
equivalence with plain multi-head attention; causality (changing later
tokens leaves earlier logits unchanged); greedy tie and threshold rules;
the affine linear against the C restatement of affine_dequantize
(oracle/oracle.py, pinned to the reference's golden vectors) and a known
answer that fails a per-flat-index or transposed group lookup.
"""
from __future__ import annotations

import numpy as np


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(w, dtype=np.float64)


def rope(x: np.ndarray, pos: np.ndarray, theta: float) -> np.ndarray:
    """x: [T, n_heads, hd]; pos: [T] integer positions."""
    hd = x.shape[-1]
    half = hd // 2
    inv_freq = theta ** (-2.0 * np.arange(half, dtype=np.float64) / hd)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv_freq[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_pos: np.ndarray | None = None) -> np.ndarray:
    """Causal GQA attention.  q [Tq, nh, hd], k/v [Tk, nkv, hd]; query i sits at
    position q_pos[i] (default Tk - Tq + i) and sees keys 0..q_pos[i]."""
    tq, nh, hd = q.shape
    tk, nkv, _ = k.shape
    grp = nh // nkv
    if q_pos is None:
        q_pos = np.arange(tk - tq, tk)
    mask = np.arange(tk)[None, :] > np.asarray(q_pos)[:, None]  # [Tq, Tk]
    out = np.empty((tq, nh, hd), dtype=np.float64)
    for h in range(nh):
        g = h // grp
        s = q[:, h, :] @ k[:, g, :].T / np.sqrt(hd)
        s = np.where(mask, -np.inf, s)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v[:, g, :]
    return out


def silu(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def linear(x: np.ndarray, qw) -> np.ndarray:
    """Per-row int8 (q, s): x . (q * s)^T with the per-row scale applied after
    the exact integer-weighted sum (equal to dequantizing first, in exact
    arithmetic).  Affine u8 (u, s, b, group): x . W^T with W[n, k] =
    u[n, k] * s[n, k // group] + b[n, k // group] (affine_dequantize,
    kernels.wgsl:379-400; b = None means zero)."""
    if len(qw) == 2:
        q, s = qw
        return (x @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
    u, s, b, group = qw
    n, k = u.shape
    rep = lambda a: np.repeat(np.asarray(a, dtype=np.float64).reshape(n, k // group), group, axis=1)  # noqa: E731
    wd = u.astype(np.float64) * rep(s) + (rep(b) if b is not None else 0.0)
    return x @ wd.T


def forward(cfg, w, tokens, first: int = 0) -> np.ndarray:
    """Logits [T - first, vocab] of positions first..T-1 of `tokens`.

    cfg: rusty_amd.llama.LlamaConfig-like; w: LlamaHostWeights-like (embed,
    layers[{attn_norm, mlp_norm, q, k, v, o, gate, up, down}], final_norm,
    lm_head)."""
    tokens = np.asarray(tokens, dtype=np.int64)
    T = tokens.size
    nh, nkv, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    pos = np.arange(T)
    x = np.asarray(w.embed, dtype=np.float64)[tokens]
    for L in w.layers:
        xn = rmsnorm(x, L["attn_norm"], cfg.norm_eps)
        q = rope(linear(xn, L["q"]).reshape(T, nh, hd), pos, cfg.rope_theta)
        k = rope(linear(xn, L["k"]).reshape(T, nkv, hd), pos, cfg.rope_theta)
        v = linear(xn, L["v"]).reshape(T, nkv, hd)
        x = x + linear(attention(q, k, v).reshape(T, nh * hd), L["o"])
        xn = rmsnorm(x, L["mlp_norm"], cfg.norm_eps)
        x = x + linear(silu(linear(xn, L["gate"])) * linear(xn, L["up"]), L["down"])
    xn = rmsnorm(x[first:], w.final_norm, cfg.norm_eps)
    return linear(xn, w.lm_head)


def greedy(logits: np.ndarray) -> int:
    """The reference's top_k scan with k = 1 (kernels.wgsl:177-186)."""
    best, idx = -1e9, 0
    for i, v in enumerate(np.asarray(logits).tolist()):
        if v > best:
            best, idx = v, i
    return idx
