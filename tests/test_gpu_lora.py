"""GPU parity of rq_qmatmul_lora: Linear::forward with a LoRA adapter
(rusty-graph/src/lib.rs:69-83), Y = X . deq(W)^T + (X . A) . B, A [in, rank],
B [rank, out], added unscaled.

* The adapter's term against the oracle's restatement of the reference's f32
  matmul (oracle/oracle.py `matmul`, one fma chain per output over k
  ascending): bit for bit, with W's term exactly zero (affine codes with zero
  scales and biases, so every kernel family's product is an exact 0).
* The whole output against the f64 truth of both terms: the fused product's
  fp16/f32 bars of the other qmatmul tests.
* rank 0 reproduces rq_qmatmul; workspace and argument errors.
"""
import numpy as np
import pytest

from conftest import f16_tol_check, f32_norm_check
from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, RqError, UnifiedTensor, synth

pytestmark = pytest.mark.gpu


def _adapter(g, k, n, rank):
    a = (g.standard_normal((k, rank)) * 0.05).astype(np.float32)
    b = (g.standard_normal((rank, n)) * 0.05).astype(np.float32)
    return a, b


# m = 1, 2 (decode GEMV), 5, 16 (MFMA GEMV), 40, 300 (GEMM)
@pytest.mark.parametrize("m", [1, 2, 5, 16, 40, 300])
@pytest.mark.parametrize("xdt", [np.float16, np.float32])
def test_adapter_term_bit_exact(ctx, engine, m, xdt):
    g = synth.rng(m * 7 + (xdt == np.float32))
    n, k, rank = 320, 512, 17
    u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
    zeros = np.zeros(n * k // 64, np.float32)
    W = QuantizedTensor.affine(ctx, u, zeros, zeros)  # deq(W) = 0 exactly
    x = synth.activations(g, m, k, dtype=xdt)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16 if xdt == np.float16 else DType.FP32)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    engine.qmatmul_lora(ctx, X, W, A, B, Y)
    want = orc.matmul(orc.matmul(x.astype(np.float32), a, fused=True), b, fused=True)
    np.testing.assert_array_equal(Y.to_vec().reshape(m, n), want)


# other ranks: past the output kernel's register-held B columns (70), and
# fp16 x at rank <= 16, where x . A's chain kernel widens x while staging
# instead of through an f32 copy
@pytest.mark.parametrize("m,rank,xdt", [(3, 70, np.float32), (300, 5, np.float32), (1, 16, np.float16),
                                        (2, 9, np.float16), (300, 16, np.float16)])
def test_adapter_term_bit_exact_ranks(ctx, engine, m, rank, xdt):
    g = synth.rng(m + rank)
    n, k = 192, 256
    u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
    zeros = np.zeros(n * k // 64, np.float32)
    W = QuantizedTensor.affine(ctx, u, zeros, zeros)  # deq(W) = 0 exactly
    x = synth.activations(g, m, k, dtype=xdt)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16 if xdt == np.float16 else DType.FP32)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    engine.qmatmul_lora(ctx, X, W, A, B, Y)
    want = orc.matmul(orc.matmul(x.astype(np.float32), a, fused=True), b, fused=True)
    np.testing.assert_array_equal(Y.to_vec().reshape(m, n), want)


@pytest.mark.parametrize("m,fmt,ydt", [(1, 0, np.float16), (4, 1, np.float32), (16, 0, np.float32),
                                       (64, 1, np.float16), (512, 0, np.float16)])
def test_full_output_against_truth(ctx, engine, m, fmt, ydt):
    g = synth.rng(100 + m + fmt)
    n, k, rank = 1024, 2048, 8
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        bi, W = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, bi = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, bi)
    x = synth.activations(g, m, k)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, ydt), dtype=DType.FP16 if ydt == np.float16 else DType.FP32)
    engine.qmatmul_lora(ctx, X, W, A, B, Y)
    x64 = x.astype(np.float64)
    truth = orc.qlinear_truth(q, s, bi, x.astype(np.float32), fmt) + (x64 @ a.astype(np.float64)) @ b.astype(np.float64)
    y = Y.to_vec().reshape(m, n)
    if ydt == np.float16:
        max_abs, rel, ok = f16_tol_check(y, truth)
    else:
        max_abs, rel, ok = f32_norm_check(y, truth, tol=2e-3)  # fp16 rounding of x inside the fused product
    print(f"[lora m={m} fmt={fmt}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_rank_zero_is_qmatmul(ctx, engine):
    g = synth.rng(5)
    n, k, m = 256, 512, 3
    q, s = synth.rowwise_weight(g, n, k)
    W = QuantizedTensor.rowwise(ctx, q, s)
    X = UnifiedTensor.new(ctx, synth.activations(g, m, k), dtype=DType.FP16)
    A = UnifiedTensor.empty(ctx, [k, 0], DType.FP32)
    B = UnifiedTensor.empty(ctx, [0, n], DType.FP32)
    Y1 = UnifiedTensor.empty(ctx, [m, n], DType.FP32)
    Y2 = UnifiedTensor.empty(ctx, [m, n], DType.FP32)
    engine.qmatmul_lora(ctx, X, W, A, B, Y1)
    engine.qmatmul(ctx, X, W, Y2)
    np.testing.assert_array_equal(Y1.to_vec(), Y2.to_vec())


def test_lora_argument_errors(ctx, engine):
    g = synth.rng(6)
    n, k, m, rank = 128, 256, 2, 4
    q, s = synth.rowwise_weight(g, n, k)
    W = QuantizedTensor.rowwise(ctx, q, s)
    X = UnifiedTensor.new(ctx, synth.activations(g, m, k), dtype=DType.FP16)
    a, b = _adapter(g, k, n, rank)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.empty(ctx, [m, n], DType.FP16)
    small = UnifiedTensor.empty(ctx, [64], DType.U8)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        engine.qmatmul_lora(ctx, X, W, A, B, Y, workspace=small)
    with pytest.raises(ValueError):
        engine.qmatmul_lora(ctx, X, W, A, UnifiedTensor.new(ctx, b[:, :64].copy()), Y)


# RQ_LORA_TREE: x . A as a fixed-order reduction tree (rq_qmatmul_lora_ex).
# With W's term exactly zero the output is the adapter's term alone, held to
# the f32 bar against the f64 truth of (x . A) . B; k_in = 300 and 5000 cut
# the 256-k slices unevenly, m = 300 and 700 take the 4-row blocks and more k
# per thread; rank 1, 17 and 64 the other widths.
@pytest.mark.parametrize("m,k,rank,xdt", [(1, 512, 16, np.float16), (2, 300, 5, np.float32), (5, 512, 17, np.float16),
                                          (16, 5000, 16, np.float16), (40, 512, 64, np.float32),
                                          (300, 300, 1, np.float16), (700, 2048, 16, np.float32)])
def test_adapter_tree_against_truth(ctx, engine, m, k, rank, xdt):
    g = synth.rng(900 + m + rank)
    n = 320
    u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
    zeros = np.zeros(-(-n * k // 64), np.float32)
    W = QuantizedTensor.affine(ctx, u, zeros, zeros)  # deq(W) = 0 exactly
    x = synth.activations(g, m, k, dtype=xdt)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16 if xdt == np.float16 else DType.FP32)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    engine.qmatmul_lora(ctx, X, W, A, B, Y, tree=True)
    y = Y.to_vec().reshape(m, n)
    truth = (x.astype(np.float64) @ a.astype(np.float64)) @ b.astype(np.float64)
    max_abs, rel, ok = f32_norm_check(y, truth, tol=1e-5)
    print(f"[lora tree m={m} k={k} rank={rank}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok
    # deterministic: a second call gives the same bits
    Y2 = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    engine.qmatmul_lora(ctx, X, W, A, B, Y2, tree=True)
    np.testing.assert_array_equal(Y2.to_vec().reshape(m, n), y)


@pytest.mark.parametrize("m,fmt,ydt", [(1, 0, np.float16), (4, 1, np.float32), (512, 0, np.float16)])
def test_tree_full_output_against_truth(ctx, engine, m, fmt, ydt):
    g = synth.rng(200 + m + fmt)
    n, k, rank = 1024, 2048, 8
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        bi, W = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, bi = synth.affine_weight(g, n, k)
        W = QuantizedTensor.affine(ctx, q, s, bi)
    x = synth.activations(g, m, k)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, ydt), dtype=DType.FP16 if ydt == np.float16 else DType.FP32)
    engine.qmatmul_lora(ctx, X, W, A, B, Y, tree=True)
    x64 = x.astype(np.float64)
    truth = orc.qlinear_truth(q, s, bi, x.astype(np.float32), fmt) + (x64 @ a.astype(np.float64)) @ b.astype(np.float64)
    y = Y.to_vec().reshape(m, n)
    if ydt == np.float16:
        max_abs, rel, ok = f16_tol_check(y, truth)
    else:
        max_abs, rel, ok = f32_norm_check(y, truth, tol=2e-3)  # fp16 rounding of x inside the fused product
    print(f"[lora tree m={m} fmt={fmt}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_tree_flag_past_rank_64_keeps_the_chain(ctx, engine):
    """Adapters wider than 64 take the chain under RQ_LORA_TREE: the
    reference's bits, as rq_qmatmul_lora gives them."""
    g = synth.rng(31)
    m, n, k, rank = 3, 192, 256, 70
    u = g.integers(0, 256, size=(n, k), dtype=np.uint8)
    zeros = np.zeros(n * k // 64, np.float32)
    W = QuantizedTensor.affine(ctx, u, zeros, zeros)
    x = synth.activations(g, m, k, dtype=np.float32)
    a, b = _adapter(g, k, n, rank)
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP32)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    engine.qmatmul_lora(ctx, X, W, A, B, Y, tree=True)
    want = orc.matmul(orc.matmul(x, a, fused=True), b, fused=True)
    np.testing.assert_array_equal(Y.to_vec().reshape(m, n), want)


def test_lora_ex_flags_and_workspace(ctx, engine):
    from rusty_amd import _lib
    g = synth.rng(32)
    n, k, m, rank = 128, 512, 2, 4
    q, s = synth.rowwise_weight(g, n, k)
    W = QuantizedTensor.rowwise(ctx, q, s)
    X = UnifiedTensor.new(ctx, synth.activations(g, m, k), dtype=DType.FP16)
    a, b = _adapter(g, k, n, rank)
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    Y = UnifiedTensor.empty(ctx, [m, n], DType.FP16)
    L = _lib.lib()
    need_tree = L.rq_qmatmul_lora_ex_workspace(m, k, n, rank, _lib.RQ_F16, _lib.RQ_F16, _lib.RQ_LORA_TREE)
    # the tree's partials: 2 slices of 256 k per row and rank, plus the f32 product
    assert need_tree >= (m * rank * 2 + m * n) * 4
    assert L.rq_qmatmul_lora_ex_workspace(m, k, n, rank, _lib.RQ_F16, _lib.RQ_F16, 0) == \
        L.rq_qmatmul_lora_workspace(m, k, n, rank, _lib.RQ_F16, _lib.RQ_F16)
    ws = UnifiedTensor.empty(ctx, [need_tree], DType.U8)
    d = W.descriptor()
    import ctypes
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul_lora_ex", ctx.handle, ctypes.byref(d), X.ptr, _lib.RQ_F16, A.ptr, B.ptr, rank, Y.ptr,
                  _lib.RQ_F16, m, 2, ws.ptr, need_tree, None)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul_lora_ex", ctx.handle, ctypes.byref(d), X.ptr, _lib.RQ_F16, A.ptr, B.ptr, rank, Y.ptr,
                  _lib.RQ_F16, m, _lib.RQ_LORA_TREE, ws.ptr, need_tree - 1, None)
    _lib.call("rq_qmatmul_lora_ex", ctx.handle, ctypes.byref(d), X.ptr, _lib.RQ_F16, A.ptr, B.ptr, rank, Y.ptr,
              _lib.RQ_F16, m, _lib.RQ_LORA_TREE, ws.ptr, need_tree, None)
    ctx.sync()
