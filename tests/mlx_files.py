"""Writes tiny Llama checkpoints in MLX's 8-bit affine safetensors layout
(U32-packed codes, scales and biases per 64-element group, config.json with a
``quantization`` block) for the loader and runner tests."""
import json

import numpy as np

from rusty_amd.loader import save_safetensors

REFERENCE_NAMES = {"o": "self_attn.out_proj", "gate": "feed_forward.w1", "up": "feed_forward.w3",
                   "down": "feed_forward.w2", "attn_norm": "operator_norm", "mlp_norm": "ffn_norm"}
MLX_NAMES = {"o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj",
             "attn_norm": "input_layernorm", "mlp_norm": "post_attention_layernorm"}


def _enc(a, dt):
    a = np.asarray(a, dtype=np.float32)
    if dt == "BF16":
        return (a.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 is valid input
    return a.astype({"F16": np.float16, "F32": np.float32}[dt])


def write_mlx_llama(path, cfg, seed=0, names="reference", tie=True, quant_embed=True, sdt="BF16", group=64,
                    files=2, embedding_norm="random"):
    """cfg: a LlamaConfig.  Codes uniform in [0, 255]; scales ~ U(0.5, 1.5) *
    0.02 / 73.3 per group and biases ~ -128 * scale, so the weights have
    std ~0.02 around zero; norm weights 1 + U(-0.1, 0.1).  Tensors are spread
    over ``files`` safetensors files.  ``embedding_norm``: "random" (norm
    weights as above), "ones" (all 1.0) or None (no model.embedding_norm)."""
    g = np.random.default_rng(seed)
    nm = dict(REFERENCE_NAMES if names == "reference" else MLX_NAMES)
    nm.update(q="self_attn.q_proj", k="self_attn.k_proj", v="self_attn.v_proj")
    tensors = {}

    def quant(name, n, k):
        u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
        s = g.uniform(0.5, 1.5, size=(n, k // group)) * (0.02 / 73.3)
        b = -128.0 * s * g.uniform(0.98, 1.02, size=s.shape)
        tensors[f"{name}.weight"] = ("U32", u.view(np.uint32))
        tensors[f"{name}.scales"] = (sdt, _enc(s, sdt))
        tensors[f"{name}.biases"] = (sdt, _enc(b, sdt))

    def norm(name):
        tensors[f"{name}.weight"] = (sdt, _enc(1.0 + g.uniform(-0.1, 0.1, cfg.hidden), sdt))

    if quant_embed:
        quant("model.embed_tokens", cfg.vocab, cfg.hidden)
    else:
        tensors["model.embed_tokens.weight"] = ("F16", g.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float16))
    for i in range(cfg.n_layers):
        pre = f"model.layers.{i}"
        norm(f"{pre}.{nm['attn_norm']}")
        norm(f"{pre}.{nm['mlp_norm']}")
        for key, (n, k) in cfg.linear_shapes().items():
            quant(f"{pre}.{nm[key]}", n, k)
    if embedding_norm == "ones":
        tensors["model.embedding_norm.weight"] = (sdt, _enc(np.ones(cfg.hidden), sdt))
    elif embedding_norm is not None:
        norm("model.embedding_norm")
    if names != "reference":
        norm("model.norm")
    if not tie:
        quant("lm_head", cfg.vocab, cfg.hidden)
    keys = list(tensors)
    for f in range(files):
        part = {k: tensors[k] for k in keys[f::files]}
        save_safetensors(path / f"model-{f + 1:05d}-of-{files:05d}.safetensors", part)
    conf = {"num_hidden_layers": cfg.n_layers, "hidden_size": cfg.hidden, "num_attention_heads": cfg.n_heads,
            "num_key_value_heads": cfg.n_kv_heads, "intermediate_size": cfg.intermediate,
            "vocab_size": cfg.vocab, "rms_norm_eps": cfg.norm_eps, "rope_theta": cfg.rope_theta,
            "max_position_embeddings": cfg.max_seq, "quantization": {"group_size": group, "bits": 8}}
    if cfg.head_dim != cfg.hidden // cfg.n_heads:
        conf["head_dim"] = cfg.head_dim
    (path / "config.json").write_text(json.dumps(conf))
    return tensors
