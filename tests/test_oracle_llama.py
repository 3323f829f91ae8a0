"""Pins of the CPU Llama restatement (oracle/llama.py) -- no GPU.

Each check is chosen so a plausible slip fails it: a sum instead of a mean in
RMSNorm, interleaved instead of rotate-half RoPE pairs or a wrong frequency
exponent, a GQA index of h % n_kv instead of h // group, a causal mask that
lets a query see later keys, or a greedy scan that keeps the last maximum.
"""
import numpy as np
import pytest

from oracle import llama as ol
from rusty_amd.llama import LlamaConfig, synth_weights


def test_rmsnorm_known_answers():
    # [3, 4]: mean square 12.5 (a sum, 25, would give [0.6, 0.8])
    y = ol.rmsnorm(np.array([[3.0, 4.0]]), np.ones(2), 0.0)
    np.testing.assert_allclose(y, [[3 / np.sqrt(12.5), 4 / np.sqrt(12.5)]], rtol=1e-15)
    # eps enters under the root: [1, 1] with eps 1 -> 1/sqrt(2)
    np.testing.assert_allclose(ol.rmsnorm(np.array([1.0, 1.0]), np.ones(2), 1.0), [2 ** -0.5] * 2, rtol=1e-15)
    # weight multiplies elementwise; eps 0 makes it scale invariant
    g = np.random.default_rng(0)
    x, w = g.standard_normal((3, 8)), g.standard_normal(8)
    np.testing.assert_allclose(ol.rmsnorm(x, w, 0.0), ol.rmsnorm(7.5 * x, w, 0.0), rtol=1e-13)
    np.testing.assert_allclose(ol.rmsnorm(x, w, 0.0) / w, ol.rmsnorm(x, np.ones(8), 0.0), rtol=1e-13)
    # rows are independent (the reference kernel's row-0-only defect is not kept)
    np.testing.assert_allclose(ol.rmsnorm(x, w, 1e-5)[1], ol.rmsnorm(x[1:2], w, 1e-5)[0], rtol=1e-15)


def test_rope_known_answers():
    # hd = 2: one pair, frequency 1; position 1 rotates [1, 0] to [cos 1, sin 1]
    r = ol.rope(np.array([[[1.0, 0.0]]]), np.array([1]), 10000.0)
    np.testing.assert_allclose(r[0, 0], [np.cos(1.0), np.sin(1.0)], rtol=1e-15)
    # hd = 4: dim 1 pairs with dim 3 (rotate-half, not 2d/2d+1) at frequency theta^(-2/4)
    x = np.zeros((1, 1, 4))
    x[0, 0, 1] = 1.0
    r = ol.rope(x, np.array([50]), 10000.0)
    np.testing.assert_allclose(r[0, 0], [0.0, np.cos(0.5), 0.0, np.sin(0.5)], atol=1e-15)
    # position 0 is the identity; each pair keeps its norm
    g = np.random.default_rng(1)
    q = g.standard_normal((5, 3, 64))
    np.testing.assert_array_equal(ol.rope(q[:1], np.array([0]), 10000.0), q[:1])
    rq = ol.rope(q, np.arange(5) * 37, 10000.0)
    np.testing.assert_allclose(np.hypot(rq[..., :32], rq[..., 32:]), np.hypot(q[..., :32], q[..., 32:]), rtol=1e-12)


def test_rope_relative_position():
    # <rope(q, m), rope(k, n)> depends on m - n only
    g = np.random.default_rng(2)
    q, k = g.standard_normal((1, 1, 64)), g.standard_normal((1, 1, 64))

    def dot(m, n):
        return float(np.sum(ol.rope(q, np.array([m]), 10000.0) * ol.rope(k, np.array([n]), 10000.0)))

    assert dot(9, 4) == pytest.approx(dot(105, 100), rel=1e-10)
    assert dot(9, 4) != pytest.approx(dot(9, 5), rel=1e-3)


def test_attention_single_and_equal_keys():
    g = np.random.default_rng(3)
    q = g.standard_normal((1, 2, 16))
    k, v = g.standard_normal((1, 1, 16)), g.standard_normal((1, 1, 16))
    np.testing.assert_allclose(ol.attention(q, k, v), np.repeat(v, 2, axis=1), rtol=1e-15)
    # equal keys: uniform weights over the visible prefix
    k = np.repeat(g.standard_normal((1, 1, 16)), 6, axis=0)
    v = g.standard_normal((6, 1, 16))
    q = g.standard_normal((6, 1, 16))
    out = ol.attention(q, k, v)
    for i in range(6):
        np.testing.assert_allclose(out[i, 0], v[: i + 1, 0].mean(axis=0), rtol=1e-12)


def test_attention_gqa_index():
    # grouped attention == multi-head attention with each KV head repeated for
    # its group (head h reads KV head h // (n_heads / n_kv))
    g = np.random.default_rng(4)
    q = g.standard_normal((5, 8, 16))
    k, v = g.standard_normal((5, 2, 16)), g.standard_normal((5, 2, 16))
    np.testing.assert_allclose(ol.attention(q, k, v),
                               ol.attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1)), rtol=1e-13)


def test_forward_causal_and_prefix_consistent():
    cfg = LlamaConfig(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=96, vocab=50,
                      max_seq=16)
    w = synth_weights(cfg, seed=5)
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 10)
    full = ol.forward(cfg, w, toks)
    changed = toks.copy()
    changed[7:] = (changed[7:] + 1) % cfg.vocab
    np.testing.assert_allclose(ol.forward(cfg, w, changed)[:7], full[:7], rtol=1e-12)
    assert not np.allclose(ol.forward(cfg, w, changed)[7], full[7])
    np.testing.assert_allclose(ol.forward(cfg, w, toks[:5], first=4)[0], full[4], rtol=1e-12)


def test_greedy_rules():
    assert ol.greedy([1.0, 3.0, 3.0, 2.0]) == 1           # first of equal maxima
    assert ol.greedy([-2e9, -1e9, -3e9]) == 0             # nothing above -1e9
    assert ol.greedy([np.nan, -5.0, np.nan, 4.0]) == 3    # NaN never wins
