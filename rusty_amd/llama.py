"""Greedy quantized-weight Llama decode on the device (``rq_llama_*`` of the C ABI).

Host mirror of the reference's ``LlamaModel`` (rusty-graph/src/lib.rs:410-436):
token embedding (fp16 table), ``n_layers`` LlamaBlocks (RMSNorm -> GQA
attention with RoPE and a KV cache -> residual add -> RMSNorm -> SwiGLU MLP ->
residual add, lib.rs:364-378), final RMSNorm and the lm_head projection, with
greedy (top-1) sampling.  Every Linear is a quantized weight read by the
fused dequant-GEMV (per-row int8, or the reference's affine u8 codes as an
MLX checkpoint holds them: ``load_mlx``); the whole step runs from captured
HIP graphs on the device (librusty_hip.so; four steps per graph launch where
a run has four), with no host round trip between tokens.

The reference has no decode loop (its LlamaModel::forward takes the ids and a
KV cache but nothing drives generation); the loop defined here is: prefill the
prompt -- every position of a chunk at once (GEMMs over the chunk's rows and a
causal prefill attention), or one position at a time through the decode step
(``set_prefill(0)``) -- then each decode step feeds the previous greedy token.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import call, rq_llama_config, rq_llama_layer, rq_llama_weights
from .engine import DType, QuantizedTensor, UnifiedTensor, WgpuContext, _stream


@dataclass(frozen=True)
class LlamaConfig:
    n_layers: int = 22
    hidden: int = 2048
    n_heads: int = 32
    n_kv_heads: int = 4
    head_dim: int = 64
    intermediate: int = 5632
    vocab: int = 32000
    max_seq: int = 640
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0

    def c_struct(self) -> rq_llama_config:
        return rq_llama_config(self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim,
                               self.intermediate, self.vocab, self.max_seq, self.norm_eps, self.rope_theta)

    def linear_shapes(self) -> dict[str, tuple[int, int]]:
        """[out, in] of each Linear of one block."""
        qw, kw = self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        return {"q": (qw, self.hidden), "k": (kw, self.hidden), "v": (kw, self.hidden), "o": (self.hidden, qw),
                "gate": (self.intermediate, self.hidden), "up": (self.intermediate, self.hidden),
                "down": (self.hidden, self.intermediate)}

    def weight_bytes(self, affine_group: int = 0) -> int:
        """Code bytes + f32 scale (and bias) bytes read by one decode step:
        per-row int8 (one scale per row), or with ``affine_group`` the
        reference's affine u8 codes (an f32 scale and bias per group)."""
        def lin(n, k):
            return n * k + (8 * n * (k // affine_group) if affine_group else 4 * n)
        per_layer = sum(lin(n, k) for n, k in self.linear_shapes().values())
        return self.n_layers * per_layer + lin(self.vocab, self.hidden)


# the 1.1B shape (22 layers, hidden 2048, 32/4 heads of 64,
# SwiGLU 5632, vocab 32000), 512 prompt + 128 generated tokens
LLAMA_1B = LlamaConfig()


@dataclass
class LlamaHostWeights:
    """Host copies: fp16 embed [V,H] and norms [H]; each Linear either per-row
    int8 as (codes int8 [out,in], scales f32 [out]) or the reference's affine
    u8 as (codes uint8 [out,in], scales f32 [out, in/group], biases f32
    [out, in/group] or None, group)."""
    embed: np.ndarray
    layers: list[dict] = field(default_factory=list)
    final_norm: np.ndarray | None = None
    lm_head: tuple[np.ndarray, np.ndarray] | None = None


def synth_weights(cfg: LlamaConfig, seed: int = 0, affine_group: int = 0) -> LlamaHostWeights:
    """Random-init weights of the architecture (no checkpoint is available).

    Linear codes uniform in [-127, 127] with per-row scales ~ U(1.36e-4, 4.09e-4):
    the dequantized weights have std ~0.02, the usual Llama init, so
    activations stay O(1) through the layers.  With ``affine_group`` every
    Linear (lm_head included) is in the reference's affine u8 format instead:
    codes uniform in [0, 255], per group of ``affine_group`` along k an f32
    scale ~ U(0.5, 1.5) * 0.02 / 73.3 and bias -128 * scale * U(0.98, 1.02)
    (an MLX checkpoint's shape of values; std ~0.02 around zero).  Norm
    weights 1 + U(-0.1, 0.1), embeddings N(0, 1); all fp16.
    """
    g = np.random.default_rng(seed)

    def linear(n, k):
        if affine_group:
            u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
            sc = g.uniform(0.5, 1.5, size=(n, k // affine_group)) * (0.02 / 73.3)
            b = (-128.0 * sc * g.uniform(0.98, 1.02, size=sc.shape)).astype(np.float32)
            return u, sc.astype(np.float32), b, affine_group
        q = g.integers(-127, 128, size=(n, k), dtype=np.int8)
        s = g.uniform(0.02 / 73.3 * 0.5, 0.02 / 73.3 * 1.5, size=n).astype(np.float32)
        return q, s

    def norm():
        return (1.0 + g.uniform(-0.1, 0.1, size=cfg.hidden)).astype(np.float16)

    w = LlamaHostWeights(embed=g.standard_normal((cfg.vocab, cfg.hidden), dtype=np.float32).astype(np.float16))
    for _ in range(cfg.n_layers):
        layer = {"attn_norm": norm(), "mlp_norm": norm()}
        for name, (n, k) in cfg.linear_shapes().items():
            layer[name] = linear(n, k)
        w.layers.append(layer)
    w.final_norm = norm()
    w.lm_head = linear(cfg.vocab, cfg.hidden)
    return w


# Weight names tried in order: the reference's (rusty-graph/src/model_builder.rs:
# 145-206: feed_forward.w1/w3/w2, self_attn.out_proj, operator_norm/ffn_norm),
# then the usual MLX Llama names.
_NAMES = {
    "q": ("self_attn.q_proj",), "k": ("self_attn.k_proj",), "v": ("self_attn.v_proj",),
    "o": ("self_attn.out_proj", "self_attn.o_proj"),
    "gate": ("feed_forward.w1", "mlp.gate_proj"), "up": ("feed_forward.w3", "mlp.up_proj"),
    "down": ("feed_forward.w2", "mlp.down_proj"),
    "attn_norm": ("operator_norm", "input_layernorm"), "mlp_norm": ("ffn_norm", "post_attention_layernorm"),
}


def load_mlx(model_dir, max_seq: int | None = None) -> tuple[LlamaConfig, LlamaHostWeights]:
    """A Llama checkpoint in MLX's 8-bit affine layout (``config.json`` +
    ``*.safetensors``) as runner inputs.

    Follows ModelBuilder (rusty-graph/src/model_builder.rs): a weight with a
    ``.scales`` tensor is quantized (load_tensor, :68-82) and its codes,
    scales and biases are kept as they are (the reference dequantizes them to
    f32; here the fused kernels read them); norms are plain tensors
    (build_rms_norm, :140-143); the final norm is ``model.norm`` or else
    ``model.embedding_norm`` (:234-240); without ``lm_head.weight`` the
    embedding is tied to the lm_head (:242-249).  The runner's embedding table
    is fp16: a quantized ``model.embed_tokens`` is dequantized on the host
    (u * s + b in f64) and rounded to fp16, norms are rounded to fp16.
    A checkpoint with ``model.embedding_norm`` has that RMSNorm applied to the
    embedding rows before the first layer (Lfm2Model::forward,
    rusty-graph/src/lfm.rs:121-122): the norm is row-wise and a lookup selects
    rows, so the table is normalised once here, in f64 from the unrounded
    rows -- x / sqrt(mean(x^2) + eps) * w -- and then rounded to fp16; the
    tied lm_head keeps the checkpoint's own codes (lfm.rs builds it from the
    raw embedding weight, model_builder.rs:242-249).  ``max_seq`` defaults to
    ``max_position_embeddings`` (else 2048), capped at the runner's 32768
    positions."""
    from pathlib import Path

    from .loader import LoaderError, QuantizationConfig, WeightsContext, load_config

    model_dir = Path(model_dir)
    conf = load_config(model_dir / "config.json")
    quant = conf.get("quantization") or QuantizationConfig()
    heads = int(conf["num_attention_heads"])
    hidden = int(conf["hidden_size"])
    cfg = LlamaConfig(
        n_layers=int(conf["num_hidden_layers"]), hidden=hidden, n_heads=heads,
        n_kv_heads=int(conf.get("num_key_value_heads") or heads),
        head_dim=int(conf.get("head_dim") or hidden // heads), intermediate=int(conf["intermediate_size"]),
        vocab=int(conf["vocab_size"]),
        max_seq=int(max_seq or min(int(conf.get("max_position_embeddings") or 2048), 32768)),
        norm_eps=float(conf.get("norm_eps", conf.get("rms_norm_eps", 1e-5))),
        rope_theta=float(conf.get("rope_theta", 10000.0)))
    wc = WeightsContext()
    files = sorted(model_dir.glob("*.safetensors"))
    if not files:
        raise LoaderError(f"{model_dir}: no .safetensors files")
    for f in files:
        wc.load_file(f)

    def quantized(name):
        if wc.get_tensor_info(f"{name}.scales") is None:
            raise LoaderError(f"{name}: the runner takes quantized Linears (no {name}.scales)")
        codes, sc, b = wc._quantized_host(name, quant)
        n, k = codes.shape
        return codes, sc.reshape(n, k // quant.group_size), b.reshape(n, k // quant.group_size), quant.group_size

    def plain(name):
        a, _ = wc.read_bytes(f"{name}.weight")
        dt = wc.get_tensor_info(f"{name}.weight")[1]
        if dt == "BF16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        if dt not in ("F32", "F16"):
            raise LoaderError(f"{name}.weight: expected F32, F16 or BF16, got {dt}")
        return a.astype(np.float32)

    def pick(prefix, key):
        for n in _NAMES[key]:
            name = f"{prefix}.{n}"
            if wc.get_tensor_info(f"{name}.weight") is not None:
                return name
        raise LoaderError(f"{prefix}: none of {', '.join(_NAMES[key])} found")

    try:
        if wc.get_tensor_info("model.embed_tokens.scales") is not None:
            codes, sc, b, gs = quantized("model.embed_tokens")
            tied = (codes, sc, b, gs)
            rep = lambda a: np.repeat(a.astype(np.float64), gs, axis=1)  # noqa: E731
            embed = codes * rep(sc) + rep(b)
        else:
            tied = None
            embed = plain("model.embed_tokens").astype(np.float64)
        embed = embed.reshape(cfg.vocab, cfg.hidden)
        if wc.get_tensor_info("model.embedding_norm.weight") is not None:
            nw = plain("model.embedding_norm").astype(np.float64)
            embed = embed / np.sqrt((embed * embed).mean(axis=1, keepdims=True) + cfg.norm_eps) * nw
        w = LlamaHostWeights(embed=embed.astype(np.float16))
        for i in range(cfg.n_layers):
            pre = f"model.layers.{i}"
            layer = {}
            for key in ("attn_norm", "mlp_norm"):
                layer[key] = plain(pick(pre, key)).astype(np.float16)
            for key in ("q", "k", "v", "o", "gate", "up", "down"):
                layer[key] = quantized(pick(pre, key))
            w.layers.append(layer)
        final = "model.norm" if wc.get_tensor_info("model.norm.weight") is not None else "model.embedding_norm"
        w.final_norm = plain(final).astype(np.float16)
        if wc.get_tensor_info("lm_head.weight") is not None:
            w.lm_head = quantized("lm_head")
        elif tied is not None:
            w.lm_head = tied
        else:
            raise LoaderError("tied lm_head needs a quantized model.embed_tokens")
    finally:
        wc.close()
    return cfg, w


class LlamaRunner:
    """Device-resident model + KV cache + captured step graphs."""

    def __init__(self, ctx: WgpuContext, cfg: LlamaConfig, weights: LlamaHostWeights):
        self.ctx, self.cfg = ctx, cfg
        self._keep = []  # device tensors the runner borrows

        def dev_f16(a):
            t = UnifiedTensor.new(ctx, np.ascontiguousarray(a, dtype=np.float16), dtype=DType.FP16)
            self._keep.append(t)
            return t.ptr

        def dev_q(lin, prepare=True):
            qt = QuantizedTensor.rowwise(ctx, *lin) if len(lin) == 2 else QuantizedTensor.affine(
                ctx, lin[0], lin[1], lin[2], group=lin[3], prepare=prepare)
            self._keep.append(qt)
            return qt.descriptor()

        layers = (rq_llama_layer * cfg.n_layers)()
        for i, lw in enumerate(weights.layers):
            L = layers[i]
            L.attn_norm = dev_f16(lw["attn_norm"])
            L.mlp_norm = dev_f16(lw["mlp_norm"])
            # q, k and v are packed into one weight by the runner, which builds
            # that weight's prefill scale table itself
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(L, name, dev_q(lw[name], prepare=name not in ("q", "k", "v")))
        self._layers = layers
        cw = rq_llama_weights(dev_f16(weights.embed), layers, dev_f16(weights.final_norm), dev_q(weights.lm_head))
        self._cfg = cfg.c_struct()
        handle = ctypes.c_void_p()
        call("rq_llama_create", ctx.handle, ctypes.byref(self._cfg), ctypes.byref(cw), ctypes.byref(handle))
        self.handle = handle

    def prefill(self, tokens, stream=None) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        call("rq_llama_prefill", self.handle, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(t.size),
             _stream(stream))

    def decode(self, n_steps: int, stream=None) -> None:
        call("rq_llama_decode", self.handle, int(n_steps), _stream(stream))

    def set_graph(self, use_graph: bool) -> None:
        """Graph launch per step (default) or direct kernel launches."""
        call("rq_llama_set_graph", self.handle, int(bool(use_graph)))

    def set_prefill(self, rows: int) -> None:
        """Positions per batched prompt chunk (a multiple of 32), or 0 for one
        position at a time through the decode step."""
        call("rq_llama_set_prefill", self.handle, int(rows))

    def tokens(self, stream=None) -> np.ndarray:
        n = ctypes.c_int32()
        call("rq_llama_tokens", self.handle, None, 0, ctypes.byref(n), _stream(stream))
        out = np.zeros(n.value, dtype=np.int32)
        call("rq_llama_tokens", self.handle, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n.value,
             ctypes.byref(n), _stream(stream))
        return out

    def logits(self, stream=None) -> np.ndarray:
        out = np.zeros(self.cfg.vocab, dtype=np.float32)
        call("rq_llama_logits", self.handle, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), _stream(stream))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None) and self.handle.value:
            _lib.lib().rq_llama_destroy(self.handle)
            self.handle = ctypes.c_void_p()
        self._keep.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
