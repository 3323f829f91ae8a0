"""GPU parity of the quantized-weight Llama decode runner (rq_llama_*) against the oracle.

The device runs the prompt through its batched prefill (or one position at a
time, set_prefill(0)), then one graph launch per generated token; the oracle
(oracle/llama.py) runs the whole sequence at once in float64 with causal
attention, teacher-forced on the device's tokens.  Checks per step:
  * logits: max|d| <= TOL * max|logits_ref| for that step;
  * greedy: the device's token has a reference logit within
    2 * TOL * max|logits_ref| of the reference maximum (a near tie may pick
    either index; anything further off is a wrong token).
TOL = 1e-2 for the small configs, 2e-2 for the 22-layer 1.1B shape: the
device rounds GEMV inputs, the attention output and the KV cache to fp16
(relative 2^-11 each), and the difference grows with depth.
"""
import numpy as np
import pytest

from oracle import llama as ol
from rusty_amd import RqError
from mlx_files import write_mlx_llama
from rusty_amd.llama import LLAMA_1B, LlamaConfig, LlamaRunner, load_mlx, synth_weights

pytestmark = pytest.mark.gpu

TINY = LlamaConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                   max_seq=96)


def check_steps(cfg, w, toks, dev_logits, n_prompt, tol, tag):
    ref = ol.forward(cfg, w, toks[: n_prompt + len(dev_logits) - 1], first=n_prompt - 1)
    assert ref.shape == dev_logits.shape
    worst = 0.0
    for i in range(ref.shape[0]):
        scale = np.abs(ref[i]).max()
        d = np.abs(dev_logits[i].astype(np.float64) - ref[i]).max() / scale
        worst = max(worst, d)
        tok = toks[n_prompt + i]
        assert ref[i][tok] >= ref[i].max() - 2 * tol * scale, f"{tag} step {i}: token {tok} is not a greedy pick"
        assert d <= tol, f"{tag} step {i}: logits rel diff {d:.3e}"
    print(f"[{tag}] steps={ref.shape[0]} worst logits rel diff {worst:.3e}", flush=True)


def run_collect(runner, prompt, steps):
    runner.prefill(prompt)
    logits = [runner.logits()]
    for _ in range(steps):
        runner.decode(1)
        logits.append(runner.logits())
    return runner.tokens(), np.stack(logits)


@pytest.mark.parametrize("cfg", [
    TINY,
    LlamaConfig(n_layers=2, hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, intermediate=384, vocab=777,
                max_seq=64),
    LlamaConfig(n_layers=1, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, intermediate=256, vocab=300,
                max_seq=300),
    LlamaConfig(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=256, vocab=300,
                max_seq=400),
    LlamaConfig(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=256, vocab=300,
                max_seq=600),
], ids=["gqa2_hd64", "mqa_hd128", "mha_long", "gqa2_hd128_long", "gqa2_hd128_600"])
def test_small_models_match_oracle(ctx, cfg):
    # the runner splits each head's attention over 1 (max_seq <= 160), 2 (<= 320), 4 (<= 480) or 8
    # blocks: these models cover 1 and 2 at head_dim 64, 1 and 4 and 8 at head_dim 128 (the 1.1B test:
    # 8 at 64); a pass covers 64 rows at head_dim 128 and 128 at 64: the 600-position model's
    # splits (75 rows) take two passes, test_attention_multi_pass covers longer ones
    w = synth_weights(cfg, seed=cfg.hidden + cfg.vocab)
    g = np.random.default_rng(11)
    n_prompt = min(40, cfg.max_seq // 2) if cfg.max_seq < 200 else 280
    prompt = g.integers(0, cfg.vocab, n_prompt)
    steps = cfg.max_seq - n_prompt  # run to full capacity
    r = LlamaRunner(ctx, cfg, w)
    toks, logits = run_collect(r, prompt, steps)
    assert toks.shape == (n_prompt + steps + 1,)
    np.testing.assert_array_equal(toks[:n_prompt], prompt)
    check_steps(cfg, w, toks, logits, n_prompt, 1e-2, f"{cfg.n_heads}/{cfg.n_kv_heads}x{cfg.head_dim}")
    # the cache is full: one more step must be refused
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        r.decode(1)
    r.close()


@pytest.mark.parametrize("cfg,names,tie", [
    (TINY, "reference", True),
    (LlamaConfig(n_layers=2, hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, intermediate=384, vocab=777,
                 max_seq=200), "mlx", False),
], ids=["reference_names_tied", "mlx_names_hd128"])
def test_mlx_checkpoint_decodes(ctx, tmp_path, cfg, names, tie):
    """An MLX 8-bit affine checkpoint (u8 codes, bf16 scale + bias per 64)
    loaded by load_mlx decodes through the runner on the affine codes
    themselves (fused norm, attention-combine and SwiGLU prologues of the
    decode GEMV), against the oracle on the same weights."""
    write_mlx_llama(tmp_path, cfg, seed=cfg.hidden, names=names, tie=tie)
    lcfg, w = load_mlx(tmp_path)
    assert lcfg == cfg and len(w.layers[0]["q"]) == 4
    g = np.random.default_rng(31)
    n_prompt = 40
    prompt = g.integers(0, cfg.vocab, n_prompt)
    r = LlamaRunner(ctx, lcfg, w)
    toks, logits = run_collect(r, prompt, cfg.max_seq - n_prompt)
    np.testing.assert_array_equal(toks[:n_prompt], prompt)
    check_steps(cfg, w, toks, logits, n_prompt, 1e-2, f"mlx {names}")
    r.close()


def test_mixed_qkv_formats_refused(ctx):
    w = synth_weights(TINY, seed=25)
    g = np.random.default_rng(26)
    n, k = TINY.linear_shapes()["k"]
    w.layers[0]["k"] = (g.integers(0, 256, (n, k), dtype=np.uint8), np.full((n, k // 64), 1e-4, np.float32),
                        np.full((n, k // 64), -128e-4, np.float32), 64)
    with pytest.raises(RqError, match="RQ_ERR_UNSUPPORTED"):
        LlamaRunner(ctx, TINY, w)


@pytest.mark.parametrize("cfg", [
    TINY,
    LlamaConfig(n_layers=2, hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, intermediate=384, vocab=500,
                max_seq=160),
], ids=["hd64", "hd128"])
def test_prefill_chunks_and_stepwise(ctx, cfg):
    """The prompt through the batched prefill in one chunk (the default), in
    chunks of 32 positions (the later chunks attend to the cache the earlier
    ones wrote) and one position at a time through the decode step: each
    against the oracle, for the prompt's last logits and up to 8 decode steps."""
    w = synth_weights(cfg, seed=cfg.hidden + 7)
    prompt = np.random.default_rng(41).integers(0, cfg.vocab, 90)
    r = LlamaRunner(ctx, cfg, w)
    for rows in (None, 32, 64, 0):
        if rows is not None:
            r.set_prefill(rows)
        toks, logits = run_collect(r, prompt, min(8, cfg.max_seq - 90))
        np.testing.assert_array_equal(toks[:90], prompt)
        check_steps(cfg, w, toks, logits, 90, 1e-2, f"prefill rows={rows} hd={cfg.head_dim}")
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        r.set_prefill(33)
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        r.set_prefill(((cfg.max_seq + 31) // 32 + 1) * 32)
    r.close()


def test_restart_and_single_token_prompt(ctx):
    w = synth_weights(TINY, seed=21)
    r = LlamaRunner(ctx, TINY, w)
    g = np.random.default_rng(22)
    p1, p2 = g.integers(0, TINY.vocab, 17), g.integers(0, TINY.vocab, 1)
    r.prefill(p1)
    r.decode(9)
    a = r.tokens()
    r.prefill(p2)  # a new sequence reuses the cache from position 0
    r.decode(5)
    b = r.tokens()
    r.prefill(p1)
    r.decode(9)
    np.testing.assert_array_equal(r.tokens(), a)
    assert b.shape == (7,) and b[0] == p2[0]
    ref = ol.forward(TINY, w, b[:6])
    for i in range(6):
        assert ref[i][b[i + 1]] >= ref[i].max() - 2e-2 * np.abs(ref[i]).max()
    r.close()


def test_step_graph_captured_at_first_graph_step(ctx):
    """The step graph is captured by the first step that runs in graph mode: a
    runner that first steps as direct launches (no graph captured yet) and
    then switches to graph steps gives the same tokens and logits, bit for
    bit, as one that used the graph from the start (the same kernels in the
    same order), and both match the oracle."""
    w = synth_weights(TINY, seed=27)
    prompt = np.random.default_rng(28).integers(0, TINY.vocab, 20)
    a = LlamaRunner(ctx, TINY, w)
    a.set_graph(False)
    ta, la = run_collect(a, prompt, 6)
    a.set_graph(True)
    extra = []
    for _ in range(4):
        a.decode(1)
        extra.append(a.logits())
    ta = a.tokens()
    a.close()
    b = LlamaRunner(ctx, TINY, w)
    tb, lb = run_collect(b, prompt, 10)
    b.close()
    np.testing.assert_array_equal(ta, tb)
    np.testing.assert_array_equal(np.concatenate([la, np.stack(extra)]).view(np.uint32), lb.view(np.uint32))
    check_steps(TINY, w, tb, lb, 20, 1e-2, "lazy graph")


def test_multi_step_graph_matches_single_steps(ctx):
    """Runs of at least four steps replay a graph that holds four consecutive
    steps (the rest of the run: the one-step graph): decoding 11 steps in one
    call (4 + 4 + 1 + 1 + 1), then 5 more (4 + 1), gives the tokens and final
    logits, bit for bit, of the same steps as direct launches one at a time."""
    w = synth_weights(TINY, seed=31)
    prompt = np.random.default_rng(32).integers(0, TINY.vocab, 17)
    a = LlamaRunner(ctx, TINY, w)
    a.prefill(prompt)
    a.decode(11)
    a.decode(5)
    ta, la = a.tokens(), a.logits()
    a.close()
    b = LlamaRunner(ctx, TINY, w)
    b.set_graph(False)
    b.prefill(prompt)
    for _ in range(16):
        b.decode(1)
    tb, lb = b.tokens(), b.logits()
    b.close()
    np.testing.assert_array_equal(ta, tb)
    np.testing.assert_array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_invalid_arguments(ctx):
    w = synth_weights(TINY, seed=23)
    r = LlamaRunner(ctx, TINY, w)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        r.prefill([1, 2, TINY.vocab])
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        r.prefill(np.zeros(TINY.max_seq + 1, dtype=np.int32))
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        r.decode(1)  # no sequence yet
    r.close()
    bad = synth_weights(TINY, seed=24)
    bad.layers[1]["down"] = bad.layers[1]["up"]  # [I, H] where [H, I] is expected
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        LlamaRunner(ctx, TINY, bad)


def test_llama_1b_128_greedy_steps(ctx):
    """1.1B shape, 512-token prompt (one batched prefill chunk), 128
    greedy decode steps; the logits of every step (the prompt's last position,
    then each generated one) and every generated token checked against the
    oracle, teacher-forced on the device's tokens."""
    cfg = LLAMA_1B
    w = synth_weights(cfg, seed=0)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 512)
    r = LlamaRunner(ctx, cfg, w)
    toks, logits = run_collect(r, prompt, 127)
    r.close()
    assert toks.shape == (640,) and logits.shape == (128, cfg.vocab)
    np.testing.assert_array_equal(toks[:512], prompt)
    check_steps(cfg, w, toks, logits, 512, 2e-2, "1B")


def test_llama_1b_affine_128_greedy_steps(ctx):
    """configs[4] on the reference's own weight format: every Linear of the
    22-layer 1.1B model (lm_head included) as affine u8 codes with an f32
    scale and bias per 64 (what rusty-loader's upload_quantized reads,
    rusty-loader/src/lib.rs:155-218); 512-token prompt through the batched
    prefill (the affine GEMMs on their load-time scale tables), then 128
    greedy steps on the affine decode GEMVs, every step's logits and token
    against the oracle."""
    cfg = LLAMA_1B
    w = synth_weights(cfg, seed=3, affine_group=64)
    assert len(w.layers[0]["gate"]) == 4 and len(w.lm_head) == 4
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 512)
    r = LlamaRunner(ctx, cfg, w)
    toks, logits = run_collect(r, prompt, 127)
    r.close()
    assert toks.shape == (640,) and logits.shape == (128, cfg.vocab)
    np.testing.assert_array_equal(toks[:512], prompt)
    check_steps(cfg, w, toks, logits, 512, 2e-2, "1B affine")


@pytest.mark.parametrize("cfg,n_prompt", [
    (LlamaConfig(n_layers=1, hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=256, vocab=300,
                 max_seq=1100), 1030),
    (LlamaConfig(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=256, vocab=300,
                 max_seq=2200), 2060),
], ids=["hd128_1100", "hd64_2200"])
def test_attention_multi_pass(ctx, cfg, n_prompt):
    """Caches long enough that each of the 8 splits per head spans more than one
    pass of the attention kernel (64 rows at head_dim 128: 129-138 rows per
    split here, three passes; 128 rows at head_dim 64: 258-275, three passes):
    the later passes' loads, the online-softmax rescale and the pass-end
    barriers, against the f64 oracle."""
    w = synth_weights(cfg, seed=cfg.max_seq)
    prompt = np.random.default_rng(cfg.max_seq).integers(0, cfg.vocab, n_prompt)
    steps = cfg.max_seq - n_prompt
    r = LlamaRunner(ctx, cfg, w)
    toks, logits = run_collect(r, prompt, steps)
    r.close()
    np.testing.assert_array_equal(toks[:n_prompt], prompt)
    check_steps(cfg, w, toks, logits, n_prompt, 1e-2, f"multi-pass {cfg.head_dim}x{cfg.max_seq}")


def _tie_model():
    """TINY with the final norm zeroed except element 0 (so the normalised row is
    xn0 at element 0 and exactly 0 elsewhere) and an lm_head whose row r has code
    q0 = +127 or -127 at k = 0 (0 elsewhere) and scale s_r: logit_r is exactly
    q0 * s_r * xn0 as the GEMV computes it, equal for rows with equal (q0, s_r)."""
    w = synth_weights(TINY, seed=31)
    fn = np.zeros(TINY.hidden, np.float16)
    fn[0] = 1.0
    w.final_norm = fn
    q = np.zeros((TINY.vocab, TINY.hidden), np.int8)
    s = np.zeros(TINY.vocab, np.float32)
    return w, q, s


def _pick(ctx, w, n_prompt=5, steps=3):
    """The prompt's pick (end of the batched prefill), then `steps` decode
    steps through the step graph: (token, logits) of the prompt, and of each
    step."""
    r = LlamaRunner(ctx, TINY, w)
    r.prefill(np.arange(1, n_prompt + 1))
    logits = r.logits()
    tok = int(r.tokens()[n_prompt])
    dec = []
    for i in range(steps):
        r.decode(1)
        dec.append((int(r.tokens()[n_prompt + 1 + i]), r.logits()))
    r.close()
    return tok, logits, dec


def _check_steps_pick(dec, ties):
    # every decode step's token is the reference pick of that step's logits; with
    # `ties`, the step's largest logit is held by several rows (exactly equal)
    for i, (tok, lg) in enumerate(dec):
        assert tok == ol.greedy(lg.astype(np.float64)), (i, tok)
        if ties:
            assert np.count_nonzero(lg == lg.max()) >= 2, (i, lg.max())


def test_greedy_pick_ties_and_threshold(ctx):
    """top_k with k = 1 as the reference scans (kernels.wgsl:173-188): the first
    index among equal maxima, and index 0 when no logit exceeds -1e9."""
    # sign of xn0 for these weights: one row with q0 = +127
    w, q, s = _tie_model()
    q[0, 0], s[0] = 127, 1.0
    w.lm_head = (q, s)
    _, lg, _ = _pick(ctx, w, steps=0)
    sgn = 1.0 if lg[0] > 0 else -1.0
    assert lg[0] != 0.0

    # exact ties: rows 300, 640 and 941 hold the largest logit (positive), rows 200
    # and 900 the same magnitude negated; every other row 0.  First index wins: 300.
    w, q, s = _tie_model()
    for r_ in (300, 640, 941):
        q[r_, 0], s[r_] = int(127 * sgn), 1e6
    for r_ in (200, 900):
        q[r_, 0], s[r_] = int(-127 * sgn), 1e6
    w.lm_head = (q, s)
    tok, lg, dec = _pick(ctx, w)
    assert lg[300] > 0 and lg[300] == lg[640] == lg[941], (lg[300], lg[640], lg[941])
    assert tok == 300, tok
    assert tok == ol.greedy(lg.astype(np.float64))
    # the decode steps: 300 again where xn0 keeps its sign, else 200 (first of 200, 900)
    _check_steps_pick(dec, ties=True)
    assert all(t in (200, 300) for t, _ in dec), [t for t, _ in dec]

    # nothing above -1e9: every logit is very negative, rows >= 100 less so than
    # rows < 100 (the largest is at 100), but all are <= -1e9, so the pick is 0
    w, q, s = _tie_model()
    q[:, 0] = int(-127 * sgn)
    s[:] = 1e12
    s[:100] = 2e12
    w.lm_head = (q, s)
    tok, lg, dec = _pick(ctx, w)
    assert lg.max() <= -1e9 and lg.argmax() == 100, (lg.max(), lg.argmax())
    assert tok == 0, tok
    assert tok == ol.greedy(lg.astype(np.float64))
    _check_steps_pick(dec, ties=False)
