"""MLX checkpoint -> runner inputs (rusty_amd.llama.load_mlx) and the oracle's
affine linear -- no GPU.

load_mlx follows the reference's ModelBuilder (rusty-graph/src/model_builder.rs):
quantized weights are those with a ``.scales`` tensor, the final norm falls back
to ``model.embedding_norm``, and without ``lm_head.weight`` the embedding is
tied to the lm_head.  ``model.embedding_norm`` is also applied to the
embedding rows before the first layer (Lfm2Model::forward,
rusty-graph/src/lfm.rs:121-122), so the runner's table holds normalised rows.  The expected values come from the writer's own tensors
and from the C restatement of affine_dequantize (oracle/oracle.py), not from
load_mlx's code.
"""
import numpy as np
import pytest

from mlx_files import write_mlx_llama
from oracle import llama as ol
from oracle import oracle as orc
from rusty_amd.llama import LlamaConfig, load_mlx
from rusty_amd.loader import LoaderError, save_safetensors

CFG = LlamaConfig(n_layers=2, hidden=128, n_heads=4, n_kv_heads=2, head_dim=32, intermediate=192, vocab=96,
                  max_seq=48)


def _widen(dt, a):
    if dt == "BF16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def _codes(words, n):
    return words.view(np.uint8).reshape(n, -1)


def test_reference_names_tied_quantized_embed(tmp_path):
    t = write_mlx_llama(tmp_path, CFG, seed=1, names="reference", tie=True, quant_embed=True, sdt="BF16")
    cfg, w = load_mlx(tmp_path)
    assert cfg == CFG
    # every Linear keeps its codes, scales and biases as stored, group 64
    for i, layer in enumerate(w.layers):
        for key, name in (("o", "self_attn.out_proj"), ("gate", "feed_forward.w1"), ("up", "feed_forward.w3"),
                          ("down", "feed_forward.w2"), ("q", "self_attn.q_proj")):
            u, s, b, grp = layer[key]
            n, k = CFG.linear_shapes()[key]
            pre = f"model.layers.{i}.{name}"
            assert grp == 64 and u.dtype == np.uint8 and u.shape == (n, k)
            np.testing.assert_array_equal(u, _codes(t[f"{pre}.weight"][1], n))
            np.testing.assert_array_equal(s, _widen("BF16", t[f"{pre}.scales"][1]).reshape(n, k // 64))
            np.testing.assert_array_equal(b, _widen("BF16", t[f"{pre}.biases"][1]).reshape(n, k // 64))
        np.testing.assert_array_equal(
            layer["mlp_norm"], _widen("BF16", t[f"model.layers.{i}.ffn_norm.weight"][1]).astype(np.float16))
    # no model.norm: the embedding norm serves as the final norm
    np.testing.assert_array_equal(w.final_norm,
                                  _widen("BF16", t["model.embedding_norm.weight"][1]).astype(np.float16))
    # tied: the lm_head is the quantized embedding
    np.testing.assert_array_equal(w.lm_head[0], _codes(t["model.embed_tokens.weight"][1], CFG.vocab))
    # the fp16 embedding table is the dequantized embedding (C restatement of
    # the reference kernel) after the embedding RMSNorm: each row divided by
    # sqrt(|row|^2 / H + eps) and scaled by the norm weight, within one fp16
    # rounding (these rows have mean square ~4e-4, so eps = 1e-5 moves them by ~1 %)
    deq = orc.affine_dequantize(_codes(t["model.embed_tokens.weight"][1], CFG.vocab),
                                _widen("BF16", t["model.embed_tokens.scales"][1]),
                                _widen("BF16", t["model.embed_tokens.biases"][1]), group=64)
    deq = deq.reshape(CFG.vocab, CFG.hidden).astype(np.float64)
    rms = np.sqrt(np.linalg.norm(deq, axis=1, keepdims=True) ** 2 / CFG.hidden + CFG.norm_eps)
    nw = _widen("BF16", t["model.embedding_norm.weight"][1]).astype(np.float64)
    assert w.embed.dtype == np.float16 and w.embed.shape == (CFG.vocab, CFG.hidden)
    np.testing.assert_allclose(w.embed.astype(np.float64), deq / rms * nw, rtol=2 ** -10, atol=1e-4)


def test_embedding_norm_applied_at_input(tmp_path):
    # all-ones norm weight: every row of the table has root mean square 1
    # (eps = 1e-5 against rows of mean square ~0.9 moves it by < 1e-5)
    write_mlx_llama(tmp_path, CFG, seed=6, tie=False, quant_embed=False, embedding_norm="ones", files=1)
    _, w = load_mlx(tmp_path)
    rms = np.sqrt((w.embed.astype(np.float64) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms, 1.0, atol=1e-3)
    # without model.embedding_norm the table is the stored one, unnormalised
    t = write_mlx_llama(tmp_path, CFG, seed=6, tie=False, quant_embed=False, embedding_norm=None, names="mlx", files=1)
    _, w = load_mlx(tmp_path)
    np.testing.assert_array_equal(w.embed, t["model.embed_tokens.weight"][1])
    # a norm that is not the identity on rows: a row scaled by 4 maps to the same normalised row
    t = write_mlx_llama(tmp_path, CFG, seed=7, tie=False, quant_embed=False, embedding_norm="random", files=1)
    tab = t["model.embed_tokens.weight"][1]
    tab[1] = (tab[0].astype(np.float32) * 4).astype(np.float16)  # exact: a power of two
    f = next(tmp_path.glob("*.safetensors"))
    save_safetensors(f, t)
    _, w = load_mlx(tmp_path)
    np.testing.assert_array_equal(w.embed[0], w.embed[1])
    assert np.abs(w.embed[0].astype(np.float32) - tab[0].astype(np.float32)).max() > 0.05


def test_mlx_names_untied_plain_embed(tmp_path):
    t = write_mlx_llama(tmp_path, CFG, seed=2, names="mlx", tie=False, quant_embed=False, sdt="F16", files=3)
    cfg, w = load_mlx(tmp_path, max_seq=40)
    assert cfg.max_seq == 40 and cfg.n_kv_heads == 2
    tab = t["model.embed_tokens.weight"][1].astype(np.float64)
    en = t["model.embedding_norm.weight"][1].astype(np.float64)
    rms = np.sqrt(np.linalg.norm(tab, axis=1, keepdims=True) ** 2 / CFG.hidden + CFG.norm_eps)
    np.testing.assert_allclose(w.embed.astype(np.float64), tab / rms * en, rtol=2 ** -10, atol=1e-4)
    # model.norm is preferred over model.embedding_norm
    np.testing.assert_array_equal(w.final_norm, t["model.norm.weight"][1])
    np.testing.assert_array_equal(w.lm_head[0], _codes(t["lm_head.weight"][1], CFG.vocab))
    np.testing.assert_array_equal(w.layers[1]["down"][0],
                                  _codes(t["model.layers.1.mlp.down_proj.weight"][1], CFG.hidden))


def test_max_seq_default_capped(tmp_path):
    import json

    write_mlx_llama(tmp_path, CFG, seed=5, files=1)
    conf = json.loads((tmp_path / "config.json").read_text())
    conf["max_position_embeddings"] = 131072
    (tmp_path / "config.json").write_text(json.dumps(conf))
    cfg, _ = load_mlx(tmp_path)
    assert cfg.max_seq == 32768
    cfg, _ = load_mlx(tmp_path, max_seq=1000)
    assert cfg.max_seq == 1000


def test_loader_errors(tmp_path):
    t = write_mlx_llama(tmp_path, CFG, seed=3, files=1)
    # a Linear stored unquantized: the runner takes quantized Linears only
    f = next(tmp_path.glob("*.safetensors"))
    name = "model.layers.0.feed_forward.w2"
    t2 = {k: v for k, v in t.items() if not k.startswith(name)}
    t2[f"{name}.weight"] = ("F16", np.zeros((CFG.hidden, CFG.intermediate), np.float16))
    save_safetensors(f, t2)
    with pytest.raises(LoaderError, match="quantized Linears"):
        load_mlx(tmp_path)
    # a missing module names the names it tried
    t3 = {k: v for k, v in t.items() if not k.startswith("model.layers.1.self_attn.out_proj")}
    save_safetensors(f, t3)
    with pytest.raises(LoaderError, match="out_proj, self_attn.o_proj"):
        load_mlx(tmp_path)


def test_oracle_affine_linear_pins():
    # known answer: rows use their own groups (a flat-index or transposed
    # lookup would mix row 0's scale into row 1)
    u = np.array([[0, 255, 1, 2], [3, 4, 5, 6]], np.uint8)
    s = np.array([[2.0, 0.5], [1.0, -1.0]])
    b = np.array([[-1.0, 0.0], [10.0, 0.25]])
    x = np.array([[1.0, 1.0, 2.0, -2.0]])
    # row 0: W = [-1, 509, 0.5, 1];  row 1: W = [13, 14, -4.75, -5.75]
    np.testing.assert_array_equal(ol.linear(x, (u, s, b, 2)), [[508.0 + 1.0 - 2.0, 27.0 - 9.5 + 11.5]])
    # biases None means zero
    np.testing.assert_array_equal(ol.linear(x, (u, s, None, 2)), [[510.0 + 1.0 - 2.0, 7.0 - 10.0 + 12.0]])
    # against the C restatement of the reference kernel at a real shape
    g = np.random.default_rng(4)
    u = g.integers(0, 256, (48, 256), dtype=np.uint8)
    s = g.uniform(0.5, 1.5, (48, 4)).astype(np.float32)
    b = g.uniform(-200, 0, (48, 4)).astype(np.float32)
    x = g.standard_normal((3, 256))
    wd = orc.affine_dequantize(u, s, b, group=64).reshape(48, 256).astype(np.float64)
    # the C path rounds each weight to f32 (relative 2^-24): a wrong group or a
    # dropped bias moves outputs by O(100), the rounding by < 1e-5 relative
    ref = x @ wd.T
    assert np.abs(ol.linear(x, (u, s, b, 64)) - ref).max() <= 1e-5 * np.abs(ref).max()
