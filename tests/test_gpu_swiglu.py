"""GPU parity of the SwiGLU MLP (rq_mlp_swiglu) against the oracle.

Reference: MLP::forward, rusty-graph/src/lib.rs:317-323 --
y = down( silu(x . gate^T) * (x . up^T) ), silu from kernels.wgsl:104-113.
The truth (oracle/oracle.c orc_swiglu_truth) is computed in f64 from the same
fp16 activations and exactly dequantized weights, with the intermediate h
rounded to fp16 as the device stores it.  Tolerance (fp16 outputs):
|dy| <= 2e-3*|y| + 2e-3*max|y| elementwise; h is checked the same way.
"""
import numpy as np
import pytest

from conftest import f16_tol_check
from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth

pytestmark = pytest.mark.gpu


def run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float16):
    G = QuantizedTensor.rowwise(ctx, wg, sg)
    U = QuantizedTensor.rowwise(ctx, wu, su)
    D = QuantizedTensor.rowwise(ctx, wd, sd)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16 if x.dtype == np.float16 else DType.FP32)
    Y = UnifiedTensor.new(ctx, np.full((x.shape[0], wd.shape[0]), np.nan, ydt),
                          dtype=DType.FP16 if ydt is np.float16 else DType.FP32)
    h = engine.mlp_swiglu(ctx, X, G, U, D, Y)
    m, inter = x.shape[0], wg.shape[0]
    return Y.to_vec(), h.to_vec().reshape(-1)[: m * inter].reshape(m, inter)


def h_truth(x, wg, sg, wu, su):
    g = orc.qlinear_truth(wg, sg, None, x.astype(np.float32), 0)
    u = orc.qlinear_truth(wu, su, None, x.astype(np.float32), 0)
    with np.errstate(over="ignore"):
        return (g / (1.0 + np.exp(-g)) * u).astype(np.float16).astype(np.float64)


def weights(g, inter, hidden):
    wg, sg = synth.rowwise_weight(g, inter, hidden)
    wu, su = synth.rowwise_weight(g, inter, hidden)
    wd, sd = synth.rowwise_weight(g, hidden, inter)
    return wg, sg, wu, su, wd, sd


@pytest.mark.parametrize("m,hidden", [(1, 1024), (2, 1024), (3, 1024), (4, 1024), (5, 1024), (8, 1024),
                                      (12, 1024), (16, 1024), (2, 4096)])
def test_swiglu_small(ctx, engine, m, hidden):
    g = synth.rng(300 + m + hidden)
    wg, sg, wu, su, wd, sd = weights(g, 200, hidden)  # 200: ragged for every row-batch size
    x = synth.activations(g, m, hidden)
    # at hidden 4096 these statistics put |y| past the fp16 range: f32 output
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float16 if hidden <= 1024 else np.float32)
    _, _, ok_h = f16_tol_check(h, h_truth(x, wg, sg, wu, su))
    assert ok_h, "intermediate h"
    truth = orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32))
    max_abs, rel, ok = f16_tol_check(y, truth)
    print(f"[swiglu m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


@pytest.mark.parametrize("m,inter,hidden", [(4, 8196, 1024), (12, 8204, 1024), (8, 5632, 256)])
def test_swiglu_row_tile_pairs(ctx, engine, m, inter, hidden):
    # 1025-1026 gate/up row tiles of 8 run two tiles per block: 8196 leaves the
    # last block's second tile empty, 8204 part-filled; hidden 256 is one
    # 256-k batch, none for the wave that finishes the second tile.  y in f32:
    # K = 8196 puts |y| past the fp16 range at these statistics
    g = synth.rng(inter + m)
    wg, sg, wu, su, wd, sd = weights(g, inter, hidden)
    x = synth.activations(g, m, hidden)
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    _, _, ok_h = f16_tol_check(h, h_truth(x, wg, sg, wu, su))
    assert ok_h, "intermediate h"
    max_abs, rel, ok = f16_tol_check(y, orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32)))
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("m", [1, 8])
def test_config3_swiglu_7b(ctx, engine, m):
    # configs[2] statistics (X ~ N(0,1), scales up to 0.02, K = 11008) put |y|
    # near 1e5, past the fp16 range: y is produced in f32 here, h stays fp16
    # (|h| < 65504 at these statistics; checked below).
    g = synth.rng(3000 + m)
    wg, sg, wu, su, wd, sd = weights(g, 11008, 4096)
    x = synth.activations(g, m, 4096)
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    ht = h_truth(x, wg, sg, wu, su)
    assert np.isfinite(ht).all() and np.isfinite(h).all()
    _, _, ok_h = f16_tol_check(h, ht)
    assert ok_h
    truth = orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32))
    max_abs, rel, ok = f16_tol_check(y, truth)
    print(f"[C3 swiglu m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_swiglu_prefill_path(ctx, engine):
    g = synth.rng(77)
    wg, sg, wu, su, wd, sd = weights(g, 384, 512)
    x = synth.activations(g, 130, 512)
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd)
    # prefill rounds g and u to fp16 before silu*mul: same tolerance
    _, _, ok_h = f16_tol_check(h, h_truth(x, wg, sg, wu, su))
    assert ok_h
    _, _, ok = f16_tol_check(y, orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32)))
    assert ok


@pytest.mark.parametrize("m,inter,hidden", [(512, 5632, 2048), (1000, 2760, 1024), (2048, 11008, 4096)],
                         ids=["1b_512", "ragged_1000x2760", "7b_2048"])
def test_swiglu_prefill_fused(ctx, engine, m, inter, hidden):
    """Gate and up through one GEMM launch with the silu*mul epilogue (enough
    tokens for the large tiles): each tile multiplies the same rows of both
    weights and writes h = silu(g) * u.  2760 intermediate rows leave the last
    tile 72 of its 128 rows per weight and 1000 tokens a partial token tile.
    h is checked on sampled rows against the f64 truth (with g and u rounded to
    fp16 as the device rounds them), y likewise (the 7B shape's full truth is
    too slow here)."""
    g = synth.rng(1000 + m)
    wg, sg, wu, su, wd, sd = weights(g, inter, hidden)
    x = synth.activations(g, m, hidden, sigma=0.5)
    # at these statistics |y| passes the fp16 range (as in the configs[2] test): y in f32
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    rows = np.unique(np.concatenate([[0, 1, m // 2, m - 2, m - 1], synth.rng(m).integers(0, m, 12)]))
    ht = h_truth(x[rows], wg, sg, wu, su)
    max_abs, rel, ok_h = f16_tol_check(h[rows], ht)
    print(f"[fused {m}x{inter}x{hidden}] h max_abs={max_abs:.3e}", flush=True)
    assert ok_h
    # a swapped gate/up half or an offset row shows in h everywhere
    assert np.isfinite(h).all()
    truth = orc.swiglu_truth(wg, sg, wu, su, wd, sd, x[rows].astype(np.float32))
    max_abs, rel, ok = f16_tol_check(y[rows], truth)
    print(f"[fused {m}x{inter}x{hidden}] y max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


@pytest.mark.parametrize("m,inter,hidden", [(1000, 2760, 1024), (768, 2816, 1024)], ids=["128x256", "128x128"])
def test_swiglu_prefill_fused_affine(ctx, engine, m, inter, hidden):
    """The fused gate/up GEMM on the reference's affine u8 weights (scale tables
    prepared at load): the tile's gate half stages its scales and offsets from
    the gate's table, the up half from the up weight's.  2760 rows leave the
    last 128x256 tile a partial half per weight.  h (against g and u rounded to
    fp16, as the kernel rounds them) and y on sampled rows against the f64
    truth."""
    g = synth.rng(1500 + m)
    ug, sg, bg = synth.affine_weight(g, inter, hidden)
    uu, su, bu = synth.affine_weight(g, inter, hidden)
    ud, sd, bd = synth.affine_weight(g, hidden, inter)
    G, U, D = (QuantizedTensor.affine(ctx, *a) for a in ((ug, sg, bg), (uu, su, bu), (ud, sd, bd)))
    x = synth.activations(g, m, hidden, sigma=0.5)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((m, hidden), np.nan, np.float32), dtype=DType.FP32)
    h = engine.mlp_swiglu(ctx, X, G, U, D, Y)
    rows = np.unique(np.concatenate([[0, 1, m // 2, m - 2, m - 1], synth.rng(m).integers(0, m, 12)]))
    xr = x[rows].astype(np.float32)
    gt = orc.qlinear_truth(ug, sg, bg, xr, 1).astype(np.float16).astype(np.float64)
    ut = orc.qlinear_truth(uu, su, bu, xr, 1).astype(np.float16).astype(np.float64)
    with np.errstate(over="ignore"):
        ht = gt / (1.0 + np.exp(-gt)) * ut
    hd = h.to_vec().reshape(-1)[: m * inter].reshape(m, inter)[rows]
    max_abs, rel, ok_h = f16_tol_check(hd, ht)
    print(f"[fused affine {m}x{inter}x{hidden}] h max_abs={max_abs:.3e}", flush=True)
    assert ok_h
    truth = orc.qlinear_truth(ud, sd, bd, ht.astype(np.float16).astype(np.float32), 1)
    max_abs, rel, ok = f16_tol_check(Y.to_vec().reshape(m, hidden)[rows], truth)
    print(f"[fused affine {m}x{inter}x{hidden}] y max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_swiglu_prefill_fused_128x128(ctx, engine):
    """1024 tokens x 2 x 2048 rows take the fused epilogue on the 128x128 tile
    (the cases above run 128x256): h and y against the f64 truth on rows at
    token-tile edges."""
    g = synth.rng(4242)
    m, inter, hidden = 1024, 2048, 1024
    wg, sg, wu, su, wd, sd = weights(g, inter, hidden)
    x = synth.activations(g, m, hidden, sigma=0.5)
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    rows = np.array([0, 127, 128, 511, 895, 1023])
    _, _, ok_h = f16_tol_check(h[rows], h_truth(x[rows], wg, sg, wu, su))
    assert ok_h and np.isfinite(h).all()
    _, _, ok = f16_tol_check(y[rows], orc.swiglu_truth(wg, sg, wu, su, wd, sd, x[rows].astype(np.float32)))
    assert ok


def test_swiglu_generic_paths(ctx, engine):
    g = synth.rng(78)
    wg, sg, wu, su, wd, sd = weights(g, 96, 100)  # K % 16 != 0: generic gate/up and down kernels
    x = synth.activations(g, 3, 100, dtype=np.float32)  # f32 activations
    y, _ = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    _, _, ok = f16_tol_check(y, orc.swiglu_truth(wg, sg, wu, su, wd, sd, x))
    assert ok


@pytest.mark.parametrize("m,inter,hidden", [(1, 1408, 2048), (2, 1408, 2048), (8, 1408, 2048), (1, 1410, 4096),
                                            (2, 1410, 4096)])
def test_swiglu_f32_activations(ctx, engine, m, inter, hidden):
    """f32 activations (the reference's dtype) through the fused gate/up passes
    (the decode kernel for 1-2 tokens, the matrix-core pass for 3-16): each value
    split into two fp16 terms, so g and u keep f32 accuracy before h is rounded.
    hidden 4096 at one or two tokens: four gate/up pairs per block, 1410
    leaving a ragged last block."""
    g = synth.rng(700 + m + hidden)
    wg, sg, wu, su, wd, sd = weights(g, inter, hidden)
    x = synth.activations(g, m, hidden, dtype=np.float32)
    y, h = run_mlp(ctx, engine, x, wg, sg, wu, su, wd, sd, ydt=np.float32)
    _, _, ok_h = f16_tol_check(h, h_truth(x, wg, sg, wu, su))
    assert ok_h, "intermediate h"
    max_abs, rel, ok = f16_tol_check(y, orc.swiglu_truth(wg, sg, wu, su, wd, sd, x))
    print(f"[swiglu f32 x m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_swiglu_shape_error(ctx, engine):
    from rusty_amd import RqError

    g = synth.rng(1)
    wg, sg, wu, su, wd, sd = weights(g, 32, 64)
    G, U = QuantizedTensor.rowwise(ctx, wg, sg), QuantizedTensor.rowwise(ctx, wu, su)
    Dbad = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, 64, 16))  # down must be [64, 32]
    X = UnifiedTensor.new(ctx, synth.activations(g, 1, 64), dtype=DType.FP16)
    Y = UnifiedTensor.empty(ctx, [1, 64], DType.FP16)
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        engine.mlp_swiglu(ctx, X, G, U, Dbad, Y)


@pytest.mark.parametrize("m,hidden,xdt", [(1, 1024, np.float16), (2, 1024, np.float16), (1, 4096, np.float16),
                                         (2, 2560, np.float16), (8, 1024, np.float16), (16, 1024, np.float16),
                                         (1, 2048, np.float32), (4, 2048, np.float32), (16, 1024, np.float32)])
def test_swiglu_affine_weights(ctx, engine, m, hidden, xdt):
    """The MLP on the reference's affine weights (u8, scale + bias per 64): gate and
    up in one pass with the silu*mul epilogue -- the decode kernel's SwiGLU pass
    for 1-2 tokens (row groups of 64/256 threads, 1-3 chunks per thread), the
    matrix-core pass for 3-16."""
    g = synth.rng(500 + m + hidden + (xdt == np.float32))
    inter = 320
    ug, sg, bg = synth.affine_weight(g, inter, hidden)
    uu, su, bu = synth.affine_weight(g, inter, hidden)
    ud, sd, bd = synth.affine_weight(g, hidden, inter)
    G, U, D = (QuantizedTensor.affine(ctx, *a) for a in ((ug, sg, bg), (uu, su, bu), (ud, sd, bd)))
    x = synth.activations(g, m, hidden, dtype=xdt)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16 if xdt == np.float16 else DType.FP32)
    Y = UnifiedTensor.new(ctx, np.full((m, hidden), np.nan, np.float32), dtype=DType.FP32)
    h = engine.mlp_swiglu(ctx, X, G, U, D, Y)
    gt = orc.qlinear_truth(ug, sg, bg, x.astype(np.float32), 1)
    ut = orc.qlinear_truth(uu, su, bu, x.astype(np.float32), 1)
    with np.errstate(over="ignore"):
        ht = (gt / (1.0 + np.exp(-gt)) * ut).astype(np.float16)
    hd = h.to_vec().reshape(-1)[: m * inter].reshape(m, inter)
    _, _, ok_h = f16_tol_check(hd, ht.astype(np.float64))
    assert ok_h, "intermediate h"
    truth = orc.qlinear_truth(ud, sd, bd, ht.astype(np.float32), 1)
    max_abs, rel, ok = f16_tol_check(Y.to_vec(), truth)
    print(f"[swiglu affine m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok
