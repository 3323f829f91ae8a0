"""GPU parity of the fused quantized linear (rq_qmatmul) against the oracle's
f64 truth of Y = X . deq(W)^T.

Tolerances (stated here, reported by every test):
  * f32 output: max|dy| / max|y| <= 1e-5
  * fp16 output: |dy| <= 2e-3*|y| + 2e-3*max|y| elementwise
The truth is computed from the same fp16-rounded X and the exactly dequantized
weight.  The configs[3] shapes are checked on every output element (per-row
codes at all three, affine codes at 4096x4096); the other full prefill sizes
on sampled rows that cover every 128-row tile and every row position inside a
tile, plus a column-checksum (sum over all tokens, a linear invariant) that
covers every output row.
"""
import numpy as np
import pytest

from conftest import f16_tol_check, f32_norm_check
from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, RqError, UnifiedTensor, synth

pytestmark = pytest.mark.gpu

F = {np.float16: DType.FP16, np.float32: DType.FP32}


def qmm(ctx, engine, w, x, ydt):
    X = UnifiedTensor.new(ctx, x, dtype=F[x.dtype.type])
    Y = UnifiedTensor.new(ctx, np.full((x.shape[0], w.n_out), np.nan, ydt), dtype=F[ydt])
    engine.qmatmul(ctx, X, w, Y)
    return Y.to_vec()


def report(name, max_abs, rel):
    print(f"[{name}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)


# ---- config 1: C1 int8 [1024,1024] x f32 [8,1024] -> f32 ----------------------

def test_config1_rowwise_f32(ctx, engine):
    g = synth.rng(0)
    q, s = synth.rowwise_weight(g, 1024, 1024)
    x = synth.activations(g, 8, 1024, dtype=np.float32)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float32)
    truth = orc.qlinear_truth(q, s, None, x, 0)
    max_abs, rel, ok = f32_norm_check(y, truth)
    ref_y, _ = orc.ref_linear(q, s, None, x, 0)  # the reference's own f32 rounding order
    report("C1 rowwise f32", max_abs, rel)
    print(f"   vs reference-order f32: max_abs={np.abs(y - ref_y).max():.3e}", flush=True)
    assert ok


def test_config1_affine_reference_format_f32(ctx, engine):
    g = synth.rng(0)
    u, s, b = synth.affine_weight(g, 1024, 1024)
    x = synth.activations(g, 8, 1024, dtype=np.float32)
    y = qmm(ctx, engine, QuantizedTensor.affine(ctx, u, s, b), x, np.float32)
    truth = orc.qlinear_truth(u, s, b, x, 1)
    max_abs, rel, ok = f32_norm_check(y, truth)
    report("C1 affine f32", max_abs, rel)
    assert ok


# ---- decode GEMV (m <= 16) ---------------------------------------------------

@pytest.mark.parametrize("m", [1, 4, 16])
def test_config2_decode_4096(ctx, engine, m):
    g = synth.rng(100 + m)
    q, s = synth.rowwise_weight(g, 4096, 4096)
    x = synth.activations(g, m, 4096)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    truth = orc.qlinear_truth(q, s, None, x.astype(np.float32), 0)
    max_abs, rel, ok = f16_tol_check(y, truth)
    report(f"C2 m={m}", max_abs, rel)
    assert ok


@pytest.mark.parametrize("k", [1024, 2048, 4096, 5632, 11008])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 12])
def test_gemv_shapes(ctx, engine, m, k):
    g = synth.rng(m * 100000 + k)
    n = 200  # not a multiple of the row batch
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("k", [16, 2064, 8208, 16400, 20480])
@pytest.mark.parametrize("m", [3, 4, 5, 9, 16])
def test_gemv_skinny_batch_counts(ctx, engine, m, k):
    # 3 <= m <= 16 runs 8 (K <= 4096) or 4 waves that each take 256-wide k
    # batches, two in flight: these K give a wave from no batch to 20 (odd and
    # even counts), and K % 256 != 0 leaves a part-live last batch whose dead
    # chunks would otherwise read the next row
    g = synth.rng(m * 7 + k)
    n = 37  # ragged last row block
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("n,k", [(16391, 2048), (20000, 1024), (16384, 5632)])
def test_gemv_tall_weights(ctx, engine, n, k):
    # n_out >= 16384 at m = 1 runs 8 rows per row group (an lm_head shape);
    # 16391 leaves a ragged last block
    g = synth.rng(n + k)
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, 1, k)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("m,n,k", [(8, 4100, 1024), (5, 8184, 2048), (16, 8200, 1024), (12, 8216, 4096),
                                   (16, 11008, 4096), (8, 4100, 64), (5, 5000, 256), (12, 8200, 128)])
def test_gemv_row_tile_pairs(ctx, engine, m, n, k):
    # 3 <= m <= 16 with 257-512 row tiles of 16 (or more than 512 at m > 8)
    # runs two tiles per block: 4100 and 8200 leave the last block's second
    # tile empty, 8184 and 8216 leave a part-filled last tile.  k <= 256 is
    # one 256-k batch: the wave that finishes the second tile has none of its
    # own (its row scales were once left unloaded)
    g = synth.rng(n * 31 + m)
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok, (max_abs, rel)


# m = 1-2: the dot2 GEMV (138 rows: not a multiple of its 4- or 8-row blocks); 3-16: the
# matrix-core GEMV (nine 16-row tiles, the last ragged; k = 11008 is 43 batches of 256)
@pytest.mark.parametrize("k", [1024, 4096, 11008])
@pytest.mark.parametrize("m", [1, 3, 4, 8, 12, 16])
def test_gemv_affine_reference_format(ctx, engine, m, k):
    g = synth.rng(m + k)
    u, s, b = synth.affine_weight(g, 138, k)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, QuantizedTensor.affine(ctx, u, s, b), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(u, s, b, x.astype(np.float32), 1))
    report(f"affine GEMV m={m} k={k}", max_abs, rel)
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("m", [5, 16])
def test_gemv_affine_4096_no_biases(ctx, engine, m):
    # the configs[1] shape in the reference's format, and biases omitted (NULL reads as 0)
    g = synth.rng(77 + m)
    u, s, _ = synth.affine_weight(g, 4096, 4096)
    x = synth.activations(g, m, 4096)
    y = qmm(ctx, engine, QuantizedTensor.affine(ctx, u, s, None), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(u, s, None, x.astype(np.float32), 1))
    report(f"affine GEMV 4096^2 m={m} no biases", max_abs, rel)
    assert ok, (max_abs, rel)


@pytest.mark.parametrize("ydt", [np.float16, np.float32])
def test_gemv_f32_output_and_activations(ctx, engine, ydt):
    g = synth.rng(42)
    q, s = synth.rowwise_weight(g, 333, 2048)
    x = synth.activations(g, 2, 2048, dtype=np.float32)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, ydt)
    truth = orc.qlinear_truth(q, s, None, x, 0)
    _, _, ok = f32_norm_check(y, truth) if ydt is np.float32 else f16_tol_check(y, truth)
    assert ok


# f32 activations, as the reference's Linear passes them, on the decode kernels
# (m <= 2: the dot2 GEMV; 3-16: the MFMA GEMV): each value is split into two
# fp16 terms (hi + lo equals it to ~2^-22) and the weights enter as exact code
# values (affine: u, with the group's scale and bias applied in f32), so the
# result keeps f32 accuracy: the f32 bar (1e-5 of max|y|).
# f32 activations outside fp16's range: every row holds a few entries of
# 1e5..3e5 (fp16 ends at 65504), so a plain fp16 hi/lo split would give inf
# and NaN rows.  The dot2 GEMV (m <= 2) scales each 16-value chunk by a power
# of two before splitting; the MFMA GEMV redoes a batch whose sums come out
# non-finite with its activations scaled by a power of two.  Checked per row
# against the f64 truth at the f32 bar (a row's error over its own max|y|).
# m = 2 also carries a row of values ~1e-6 (below fp16's normal range), which
# the per-chunk scaling keeps at f32 accuracy.
@pytest.mark.parametrize("m,fmt", [(1, 0), (2, 0), (4, 0), (12, 0), (1, 1), (2, 1), (4, 1), (12, 1)])
def test_f32_activations_past_fp16_range(ctx, engine, m, fmt):
    g = synth.rng(950 + 16 * m + fmt)
    n, k = 1024, 4096
    x = synth.activations(g, m, k, dtype=np.float32)
    for r in range(m):
        j = g.choice(k, size=3, replace=False)
        x[r, j] = (g.choice([-1.0, 1.0], 3) * g.uniform(1e5, 3e5, 3)).astype(np.float32)
    if m == 2:
        x[1] = (synth.activations(g, 1, k, dtype=np.float32)[0] * 1e-6).astype(np.float32)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        b, W = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, b = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, b)
    truth = orc.qlinear_truth(q, s, b, x, fmt)
    y = qmm(ctx, engine, W, x, np.float32)
    assert np.isfinite(y).all()
    for r in range(m):
        max_abs, rel, ok = f32_norm_check(y[r], truth[r])
        report(f"f32 x wide range m={m} row {r} fmt={fmt}", max_abs, rel)
        assert ok


@pytest.mark.parametrize("m,n,k,fmt", [(1, 4096, 4096, 0), (2, 4096, 4096, 0), (3, 1000, 2048, 0),
                                       (4, 4096, 4096, 0), (8, 1024, 1024, 0), (16, 4096, 4096, 0),
                                       (5, 333, 4096, 0), (1, 11008, 4096, 0), (1, 4096, 11008, 0),
                                       (1, 4096, 4096, 1), (2, 1000, 2048, 1), (3, 1000, 2048, 1),
                                       (4, 4096, 4096, 1), (8, 1024, 1024, 1), (16, 4096, 4096, 1),
                                       (11, 333, 4096, 1), (1, 11004, 4096, 0), (1, 4100, 8192, 1),
                                       (1, 4098, 4096, 0), (2, 4100, 4096, 0), (2, 4100, 4096, 1)])
def test_f32_activations_decode_kernels(ctx, engine, m, n, k, fmt):
    g = synth.rng(900 + m + n + fmt)
    x = synth.activations(g, m, k, dtype=np.float32)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        b, W = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, b = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, b)
    truth = orc.qlinear_truth(q, s, b, x, fmt)
    y = qmm(ctx, engine, W, x, np.float32)
    max_abs, rel, ok = f32_norm_check(y, truth)
    report(f"f32 x m={m} {n}x{k} fmt={fmt} -> f32", max_abs, rel)
    assert ok
    y16 = qmm(ctx, engine, W, x, np.float16)
    max_abs, rel, ok = f16_tol_check(y16, truth)
    report(f"f32 x m={m} {n}x{k} fmt={fmt} -> f16", max_abs, rel)
    assert ok


def test_swiglu_shapes_m8(ctx, engine):
    g = synth.rng(3)
    for n, k in ((11008, 4096), (4096, 11008)):
        q, s = synth.rowwise_weight(g, n, k)
        x = synth.activations(g, 8, k)
        y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
        max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
        report(f"swiglu-shape {n}x{k} m=8", max_abs, rel)
        assert ok


# ---- prefill GEMM (MFMA) -------------------------------------------------------

def _sample_rows(m, tile=128, per_tile=8):
    rows = set()
    for b in range(-(-m // tile)):
        for j in range(per_tile):
            r = b * tile + (b * per_tile + j) % tile
            if r < m:
                rows.add(r)
    rows.update({0, m - 1})
    return np.array(sorted(rows))


def _check_prefill(y, x, q, s, name):
    rows = _sample_rows(x.shape[0])
    truth = orc.qlinear_truth(q, s, None, x[rows].astype(np.float32), 0)
    max_abs, rel, ok = f16_tol_check(y[rows], truth)
    report(f"{name} sampled {len(rows)} rows", max_abs, rel)
    assert ok
    # column checksum over all tokens: sum_m Y[m, n] = (sum_m X[m, :]) . w[n, :]
    xsum = x.astype(np.float64).sum(axis=0, keepdims=True)
    col_truth = orc.qlinear_truth(q, s, None, xsum.astype(np.float32), 0)[0]
    xsum_err = np.abs(xsum - xsum.astype(np.float32).astype(np.float64))  # f32 rounding of the summed X
    w_abs = np.abs(q.astype(np.float64)) * s[:, None].astype(np.float64)
    col_dev = y.astype(np.float64).sum(axis=0)
    # fp16 output rounding of each element is <= 2^-11 |y|, independent across tokens
    sigma = np.sqrt(((2.0 ** -11 * y.astype(np.float64)) ** 2).sum(axis=0) / 3)
    bound = 8 * sigma + w_abs @ xsum_err[0] + 1e-5 * np.abs(y.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(col_dev - col_truth) <= bound), float((np.abs(col_dev - col_truth) / bound).max())


# configs[3] at full size, every output element against the f64 truth (the
# exactly dequantized weight, W = q * s or u * s + b in f64, multiplied by the
# fp16-rounded activations with f64 BLAS), per-row codes at the three shapes
# and the reference's affine codes at 4096x4096.
@pytest.mark.parametrize("n,k,fmt", [(4096, 4096, 0), (11008, 4096, 0), (4096, 11008, 0), (4096, 4096, 1)])
def test_config4_prefill_every_element(ctx, engine, n, k, fmt):
    g = synth.rng(7000 + n + k + fmt)
    x = synth.activations(g, 2048, k, sigma=0.5)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        W = QuantizedTensor.rowwise(ctx, q, s)
        wd = q.astype(np.float64) * s.astype(np.float64)[:, None]
    else:
        q, s, b = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, b)
        rep = lambda a: np.repeat(a.astype(np.float64).reshape(n, k // 64), 64, axis=1)  # noqa: E731
        wd = q.astype(np.float64) * rep(s) + rep(b)
    y = qmm(ctx, engine, W, x, np.float16)
    truth = x.astype(np.float64) @ wd.T
    del wd
    max_abs, rel, ok = f16_tol_check(y, truth)
    report(f"C4 every element 2048x{n}x{k} fmt={fmt}", max_abs, rel)
    assert ok


@pytest.mark.parametrize("n,k", [(4096, 4096), (11008, 4096), (4096, 11008)])
def test_config4_prefill(ctx, engine, n, k):
    g = synth.rng(n + k)
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, 2048, k, sigma=0.5)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    assert np.isfinite(y).all()
    _check_prefill(y, x, q, s, f"C4 2048x{n}x{k}")


# tile per shape on a 256-CU device: 64x64 for the first, second and fourth, 128x64 for
# (300, 4096), 128x128 (two k-groups of 4 waves, weight staged in pairs of k-steps) for
# (770, 4096) and (1100, 4100), 128x256 (the same) for (1500, 4100); k = 1088 is 17 k-steps, not a
# multiple of the LDS ring period, and odd (the last weight pair is half past the k range)
@pytest.mark.parametrize("m,n,k", [(17, 300, 1024), (200, 136, 2048), (300, 4096, 64), (129, 129, 128),
                                   (770, 4096, 128), (1500, 4100, 64), (1100, 4100, 1088), (1500, 4100, 1088)])
def test_gemm_ragged(ctx, engine, m, n, k):
    g = synth.rng(m + n + k)
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok, (max_abs, rel)


# Split-K (tile grids covering at most half of a 256-CU device): 17 and 64 tokens at 4096x4096
# (64 tiles of 64x64, 4 splits of 16 k-steps), 30 tokens at 1000x11008 (16 tiles, 16 splits of
# 11 k-steps, the last of 7), 100 tokens at 1000x1088 (32 tiles; 17 k-steps allow 2 splits of at
# least 8: 9 and 8).  The last block
# of a tile adds the splits in order, so a repeated call must agree bit for bit; f32 output included.
@pytest.mark.parametrize("m,n,k,ydt", [(17, 4096, 4096, np.float16), (64, 4096, 4096, np.float32),
                                       (30, 1000, 11008, np.float16), (100, 1000, 1088, np.float16)])
def test_gemm_split_k(ctx, engine, m, n, k, ydt):
    g = synth.rng(m + n + k + 3)
    q, s = synth.rowwise_weight(g, n, k)
    x = synth.activations(g, m, k, sigma=0.5)
    w = QuantizedTensor.rowwise(ctx, q, s)
    y = qmm(ctx, engine, w, x, ydt)
    assert np.isfinite(y).all()
    assert np.array_equal(y.view(np.uint8), qmm(ctx, engine, w, x, ydt).view(np.uint8)), "repeat differs"
    max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    report(f"split-K {m}x{n}x{k}", max_abs, rel)
    assert ok


# ---- the reference's own inputs on the MFMA GEMM: affine weights, f32 activations ------
# Affine u8 codes with a scale and bias per group of 64 (128) along k (the MLX format the
# reference loads, kernels.wgsl:379-400) are expanded to fp16 u*s + b with one rounding;
# f32 activations are cast to fp16 (round to nearest even) before the GEMM.  Both are then
# the fp16-MFMA path, held to the fp16 bar against the f64 truth of the unrounded inputs:
# |dy| <= 2e-3*|y| + 2e-3*max|y| (fp16 rounding of a weight or an activation is 2^-12
# relative).  Full-size checks use sampled rows plus the all-token column checksum.

def _affine(g, n, k, group=64):
    u, s, b = synth.affine_weight(g, n, k, group)
    return u, s, b


def _check_rows(y, x, w_args, name):
    rows = _sample_rows(x.shape[0])
    truth = orc.qlinear_truth(*w_args[:3], x[rows].astype(np.float32), *w_args[3:])
    max_abs, rel, ok = f16_tol_check(y[rows], truth)
    report(f"{name} sampled {len(rows)} rows", max_abs, rel)
    assert ok
    xsum = x.astype(np.float64).sum(axis=0, keepdims=True)
    col_truth = orc.qlinear_truth(*w_args[:3], xsum.astype(np.float32), *w_args[3:])[0]
    col_dev = y.astype(np.float64).sum(axis=0)
    # per-element deviations of the sampled rows, independent across tokens, bound the sum
    dev_rms = np.sqrt(((y[rows].astype(np.float64) - truth) ** 2).mean(axis=0))
    bound = 8 * np.sqrt(x.shape[0]) * dev_rms + 2e-3 * np.abs(col_truth) + 1e-3 * np.abs(col_truth).max()
    assert np.all(np.abs(col_dev - col_truth) <= bound), float((np.abs(col_dev - col_truth) / bound).max())


@pytest.mark.parametrize("xdt", [np.float16, np.float32])
def test_config4_prefill_affine(ctx, engine, xdt):
    g = synth.rng(4242)
    u, s, b = _affine(g, 4096, 4096)
    x = synth.activations(g, 2048, 4096, sigma=0.5, dtype=xdt)
    y = qmm(ctx, engine, QuantizedTensor.affine(ctx, u, s, b), x, np.float16)
    assert np.isfinite(y).all()
    _check_rows(y, x, (u, s, b, 1, 64), f"C4 affine g64 2048x4096x4096 x={np.dtype(xdt).name}")


# The scale table built once per weight at load (rq_qweight_prepare, what
# QuantizedTensor.affine does by default) is the table the GEMM otherwise
# builds in the context's preparation area on every call: the two give the
# same bits.  A prepared weight needs no context area, so with fp16
# activations it also runs the fast GEMM on another stream (the same bits
# where the context stream does not split K).
@pytest.mark.parametrize("m,n,k,group", [(2048, 4096, 4096, 64), (300, 4096, 1024, 128), (17, 300, 1024, 64),
                                         (1500, 4100, 1088, 64)])
def test_affine_prepared_table_matches_per_call(ctx, engine, m, n, k, group):
    from rusty_amd.hiprt import Stream

    g = synth.rng(5000 + m + k + group)
    u, s, b = _affine(g, n, k, group)
    x = synth.activations(g, m, k, sigma=0.5)
    wp = QuantizedTensor.affine(ctx, u, s, b, group)
    wn = QuantizedTensor.affine(ctx, u, s, b, group, prepare=False)
    assert wp.prep is not None and wp.prep.numel * 4 == 8 * n * (k // group) and wn.prep is None
    yp = qmm(ctx, engine, wp, x, np.float16)
    yn = qmm(ctx, engine, wn, x, np.float16)
    np.testing.assert_array_equal(yp.view(np.uint16), yn.view(np.uint16))
    if m >= 256:  # no split-K on the context stream either
        st = Stream()
        X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
        Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float16), dtype=DType.FP16)
        engine.qmatmul(ctx, X, wp, Y, stream=st.h)
        st.synchronize()
        np.testing.assert_array_equal(Y.to_vec().view(np.uint16), yp.view(np.uint16))
    _check_rows(yp, x, (u, s, b, 1, group), f"prepared affine {m}x{n}x{k} g={group}")


def test_qweight_prepare_arguments(ctx):
    import ctypes

    from rusty_amd import _lib

    g = synth.rng(5100)
    q, s = synth.rowwise_weight(g, 64, 256)
    wr = QuantizedTensor.rowwise(ctx, q, s)
    d = wr.descriptor()
    assert _lib.lib().rq_qweight_prep_bytes(ctypes.byref(d)) == 0  # per-row: nothing to prepare
    _lib.call("rq_qweight_prepare", ctx.handle, ctypes.byref(d), None, 0, None)
    assert not d.prep
    u, s, b = _affine(g, 64, 256)
    wa = QuantizedTensor.affine(ctx, u, s, b, prepare=False)
    d = wa.descriptor()
    assert _lib.lib().rq_qweight_prep_bytes(ctypes.byref(d)) == 8 * 64 * 4
    t = UnifiedTensor.empty(ctx, [511], DType.FP32)
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        _lib.call("rq_qweight_prepare", ctx.handle, ctypes.byref(d), t.ptr, 511 * 4, None)
    assert not d.prep
    # group 16 serves the decode kernels only: nothing to prepare
    u, s, b = _affine(g, 64, 256, 16)
    d = QuantizedTensor.affine(ctx, u, s, b, 16).descriptor()
    assert _lib.lib().rq_qweight_prep_bytes(ctypes.byref(d)) == 0 and not d.prep
    # a table on a per-row weight is refused
    d = wr.descriptor()
    d.prep = t.ptr
    Y = UnifiedTensor.empty(ctx, [1, 64], DType.FP32)
    X = UnifiedTensor.new(ctx, synth.activations(g, 1, 256), dtype=DType.FP16)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul", ctx.handle, ctypes.byref(d), X.ptr, _lib.RQ_F16, Y.ptr, _lib.RQ_F32, 1, None)


def test_config4_prefill_f32_activations(ctx, engine):
    g = synth.rng(4243)
    q, s = synth.rowwise_weight(g, 4096, 4096)
    x = synth.activations(g, 2048, 4096, sigma=0.5, dtype=np.float32)
    y = qmm(ctx, engine, QuantizedTensor.rowwise(ctx, q, s), x, np.float16)
    assert np.isfinite(y).all()
    _check_rows(y, x, (q, s, None, 0), "C4 rowwise 2048x4096x4096 x=float32")


# f32 activations past fp16's range on the GEMM path (m > 16): each row is cast
# with its own power-of-two scale (largest magnitude in [2^14, 2^15)) that the
# epilogue multiplies back, so rows with entries of 1e5..3e5 (fp16 ends at
# 65504) and a row of values ~1e-6 (below fp16's normal range) are held to the
# fp16 bar of their own rows against the f64 truth of the f32 input;
# 300 tokens: 128x64 tiles, 40 tokens: split-K 64x64 tiles.
@pytest.mark.parametrize("m,n,k,fmt", [(300, 1024, 4096, 0), (40, 4096, 4096, 0), (300, 1024, 4096, 1)])
def test_gemm_f32_activations_past_fp16_range(ctx, engine, m, n, k, fmt):
    g = synth.rng(9100 + m + fmt)
    x = synth.activations(g, m, k, sigma=0.5, dtype=np.float32)
    for r in range(0, m, 3):
        j = g.choice(k, size=3, replace=False)
        x[r, j] = (g.choice([-1.0, 1.0], 3) * g.uniform(1e5, 3e5, 3)).astype(np.float32)
    x[1] = (x[1] * 1e-6).astype(np.float32)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        b, W = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, b = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, b)
    truth = orc.qlinear_truth(q, s, b, x, fmt)
    y = qmm(ctx, engine, W, x, np.float32)
    assert np.isfinite(y).all()
    worst = 0.0
    for r in range(m):
        max_abs, rel, ok = f16_tol_check(y[r], truth[r])
        worst = max(worst, max_abs / np.abs(truth[r]).max())
        assert ok, (r, max_abs, rel)
    report(f"f32 x past fp16 range {m}x{n}x{k} fmt={fmt}: worst row max|dy|/max|y|", worst, worst)


# every tile, split-K, group 128, and f32 activations in two chunks of the preparation area
# (3000 x 16384 f32 -> fp16 is 98 MB: two chunks)
@pytest.mark.parametrize("m,n,k,fmt,group,xdt", [
    (17, 300, 1024, 1, 64, np.float16),     # 64x64, split-K
    (9, 4096, 4096, 1, 64, np.float32),     # 9 tokens, f32: the GEMM (split-K)
    (100, 1000, 1088, 1, 64, np.float32),   # 64x64, 17 k-steps
    (300, 4096, 1024, 1, 128, np.float16),  # 128x64, group 128
    (770, 4096, 128, 1, 64, np.float32),    # 128x128 pairs
    (1500, 4100, 1088, 1, 64, np.float16),  # 128x256 pairs, odd k-step count
    (1500, 4100, 1024, 0, 0, np.float32),   # rowwise, f32 activations
    (300, 512, 6144, 0, 0, np.float32),     # f32 rows cast from 4 chunks per thread
    (130, 256, 20480, 0, 0, np.float32),    # f32 rows too long to hold: read twice
    (3000, 256, 16384, 0, 0, np.float32),   # two chunks
    (3000, 256, 16384, 1, 64, np.float32),  # two chunks, affine
])
def test_gemm_affine_f32_shapes(ctx, engine, m, n, k, fmt, group, xdt):
    g = synth.rng(m * 7 + n + k + fmt)
    if fmt == 1:
        u, s, b = _affine(g, n, k, group)
        w, args = QuantizedTensor.affine(ctx, u, s, b, group), (u, s, b, 1, group)
    else:
        q, s = synth.rowwise_weight(g, n, k)
        w, args = QuantizedTensor.rowwise(ctx, q, s), (q, s, None, 0)
    x = synth.activations(g, m, k, sigma=0.5, dtype=xdt)
    y = qmm(ctx, engine, w, x, np.float32)
    assert np.isfinite(y).all()
    if m * k <= 2_000_000:
        max_abs, rel, ok = f16_tol_check(y, orc.qlinear_truth(*args[:3], x.astype(np.float32), *args[3:]))
        report(f"{m}x{n}x{k} fmt={fmt} g={group} x={np.dtype(xdt).name}", max_abs, rel)
        assert ok
    else:
        _check_rows(y, x, args, f"{m}x{n}x{k} fmt={fmt} g={group} x={np.dtype(xdt).name}")


# ---- generic path, edge cases, errors -------------------------------------------

@pytest.mark.parametrize("m,n,k,fmt", [(1, 50, 1000, 0), (3, 7, 33, 0), (20, 31, 100, 0), (2, 40, 96, 1),
                                       (64, 64, 4096, 1)])
def test_generic_path(ctx, engine, m, n, k, fmt):
    g = synth.rng(m * n + k)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        b = None
        w = QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, b = synth.affine_weight(g, n, k)
        w = QuantizedTensor.affine(ctx, q, s, b)
    x = synth.activations(g, m, k)
    y = qmm(ctx, engine, w, x, np.float32)
    _, rel, ok = f16_tol_check(y, orc.qlinear_truth(q, s, b, x.astype(np.float32), fmt))
    assert ok, rel


def test_unaligned_activation_pointer(ctx, engine):
    g = synth.rng(9)
    q, s = synth.rowwise_weight(g, 64, 1024)
    x = synth.activations(g, 1, 1024)
    X = UnifiedTensor.new(ctx, np.concatenate([np.zeros(1, np.float16), x.ravel()]), dtype=DType.FP16)
    xv = UnifiedTensor(ctx, X.ptr + 2, [1, 1024], DType.FP16, owner=False)
    Y = UnifiedTensor.empty(ctx, [1, 64], DType.FP16)
    engine.qmatmul(ctx, xv, QuantizedTensor.rowwise(ctx, q, s), Y)
    _, _, ok = f16_tol_check(Y.to_vec(), orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
    assert ok


def test_zero_k_gives_zero(ctx, engine):
    w = QuantizedTensor.rowwise(ctx, np.zeros((5, 0), np.int8), np.ones(5, np.float32))
    X = UnifiedTensor.empty(ctx, [2, 0], DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((2, 5), 7.0, np.float16), dtype=DType.FP16)
    engine.qmatmul(ctx, X, w, Y)
    assert np.all(Y.to_vec() == 0)


def test_invalid_weight_format_raises(ctx, engine):
    w = QuantizedTensor.rowwise(ctx, np.zeros((4, 16), np.int8), np.ones(4, np.float32))
    w.format = 7
    X = UnifiedTensor.empty(ctx, [1, 16], DType.FP16)
    Y = UnifiedTensor.empty(ctx, [1, 4], DType.FP16)
    with pytest.raises(RqError, match="INVALID_ARGUMENT"):
        engine.qmatmul(ctx, X, w, Y)
