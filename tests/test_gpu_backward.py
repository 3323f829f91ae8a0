"""Input gradient through a frozen quantized Linear (rq_qmatmul_dx), GPU.

With f32 dY and dX the result must equal, bit for bit, the oracle's
k-ascending fused f32 matmul of dY with the oracle-dequantized weight -- the
reference's `grad_a = matmul_bt(grad, W_f32[in, out])` (MatMulNode::backward,
rusty-autograd/src/lib.rs:152-158), written in the [out, in] orientation.
fp16 operands are checked against the f64 truth with the fp16 tolerance
|d| <= 2e-3*|y| + 2e-3*max|y|.
"""
import numpy as np
import pytest

from conftest import f16_tol_check
from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, RqError, UnifiedTensor, synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("m,n_out,k_in", [(1, 64, 64), (37, 200, 96), (130, 1024, 512), (64, 4096, 1000)])
@pytest.mark.parametrize("fmt", ["rowwise", "affine"])
def test_dx_bit_exact_f32(ctx, engine, m, n_out, k_in, fmt):
    g = synth.rng(m + n_out + k_in)
    if fmt == "rowwise":
        q, s = synth.rowwise_weight(g, n_out, k_in)
        w, wdeq = QuantizedTensor.rowwise(ctx, q, s), orc.rowwise_dequantize(q, s)
    else:
        grp = 8 if k_in % 64 else 64
        u, s, b = synth.affine_weight(g, n_out, k_in, group=grp)
        w = QuantizedTensor.affine(ctx, u, s, b, group=grp)
        wdeq = orc.affine_dequantize(u, s, b, group=grp).reshape(n_out, k_in)
    dy = g.standard_normal((m, n_out), dtype=np.float32)
    dx = UnifiedTensor.empty(ctx, [m, k_in], DType.FP32)
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy), w, dx)
    want = orc.matmul(dy, wdeq.reshape(n_out, k_in), fused=True)
    got = dx.to_vec()
    assert np.array_equal(bits(got), bits(want)), f"{np.count_nonzero(bits(got) != bits(want))} elements differ"


def test_dx_fp16(ctx, engine):
    g = synth.rng(5)
    q, s = synth.rowwise_weight(g, 768, 512)
    w = QuantizedTensor.rowwise(ctx, q, s)
    dy = synth.activations(g, 50, 768)  # fp16
    dx = UnifiedTensor.empty(ctx, [50, 512], DType.FP16)
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy, dtype=DType.FP16), w, dx)
    truth = dy.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64)[:, None])
    max_abs, rel, ok = f16_tol_check(dx.to_vec(), truth)
    print(f"[dx fp16] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_dx_is_transpose_of_forward(ctx, engine):
    # <dy, x . deq(W)^T> == <dy . deq(W), x>: the forward and the input
    # gradient use the same weight and orientation
    g = synth.rng(6)
    q, s = synth.rowwise_weight(g, 300, 256)
    w = QuantizedTensor.rowwise(ctx, q, s)
    # f32 activations at 20 tokens take the fp16 MFMA GEMM (cast on the device):
    # values representable in fp16 keep that cast exact, so both sides are f32-accurate
    x = g.standard_normal((20, 256), dtype=np.float32).astype(np.float16).astype(np.float32)
    dy = g.standard_normal((20, 300), dtype=np.float32)
    y = UnifiedTensor.empty(ctx, [20, 300], DType.FP32)
    engine.qmatmul(ctx, UnifiedTensor.new(ctx, x), w, y)
    dx = UnifiedTensor.empty(ctx, [20, 256], DType.FP32)
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy), w, dx)
    lhs = float(np.sum(dy.astype(np.float64) * y.to_vec()))
    rhs = float(np.sum(dx.to_vec().astype(np.float64) * x))
    assert lhs == pytest.approx(rhs, rel=1e-4)


def test_dx_errors(ctx, engine):
    g = synth.rng(7)
    w = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, 32, 16))
    with pytest.raises(ValueError):
        engine.qmatmul_dx(ctx, UnifiedTensor.empty(ctx, [2, 31]), w, UnifiedTensor.empty(ctx, [2, 16]))
    from rusty_amd import _lib
    import ctypes
    d = w.descriptor()
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul_dx", ctx.handle, ctypes.byref(d), None, 0, None, 0, 3, None)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul_dx", ctx.handle, ctypes.byref(d), None, 7, None, 0, 3, None)


# ---- rq_qmatmul_dx_mfma: the same gradient on the matrix cores -------------
# Held to the f32 bar against the f64 truth dY . (q s): max|d| / max|dX| <= 1e-5.
# Shapes: the GEMM's 64x64 split-K tiles (m = 1, 40), 128x64 / 128x128 tiles
# (m = 300, 512), n_out = 96 (two halves of 96 codes: 192 per transposed row,
# three 64-code steps), k_in = 48 (one partial 64-row tile of the transpose).
@pytest.mark.parametrize("m,n_out,k_in", [(1, 4096, 4096), (40, 96, 48), (300, 1024, 512), (512, 2048, 1024)])
@pytest.mark.parametrize("dyt", [np.float32, np.float16])
def test_dx_mfma_against_truth(ctx, engine, m, n_out, k_in, dyt):
    from conftest import f32_norm_check
    g = synth.rng(40 + m + n_out)
    q, s = synth.rowwise_weight(g, n_out, k_in)
    w = QuantizedTensor.rowwise(ctx, q, s)
    dy = g.standard_normal((m, n_out), dtype=np.float32).astype(dyt)
    dx = UnifiedTensor.new(ctx, np.full((m, k_in), np.nan, np.float32))
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy, dtype=DType.FP32 if dyt == np.float32 else DType.FP16), w, dx,
                      mfma=True)
    truth = dy.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64)[:, None])
    max_abs, rel, ok = f32_norm_check(dx.to_vec(), truth, tol=1e-5)
    print(f"[dx mfma m={m} n={n_out} k={k_in}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_dx_mfma_rows_past_fp16_range_and_tiny(ctx, engine):
    """dY rows of 1e5-3e5 (past fp16) and of 1e-6, each under its own power
    of two: every row to the f32 bar of its own maximum."""
    g = synth.rng(41)
    m, n_out, k_in = 6, 512, 256
    q, s = synth.rowwise_weight(g, n_out, k_in)
    w = QuantizedTensor.rowwise(ctx, q, s)
    dy = g.standard_normal((m, n_out), dtype=np.float32)
    dy[1] *= 2e5
    dy[3] *= 1e-6
    dy[4] = 0.0
    dx = UnifiedTensor.empty(ctx, [m, k_in], DType.FP32)
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy), w, dx, mfma=True)
    truth = dy.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64)[:, None])
    got = dx.to_vec()
    for i in range(m):
        if not truth[i].any():
            assert not got[i].any()
            continue
        _, rel, ok = __import__("conftest").f32_norm_check(got[i], truth[i], tol=1e-5)
        assert ok, (i, rel)


def test_dx_mfma_fp16_out_and_table_reuse(ctx, engine):
    g = synth.rng(42)
    q, s = synth.rowwise_weight(g, 768, 512)
    w = QuantizedTensor.rowwise(ctx, q, s)
    truthw = q.astype(np.float64) * s.astype(np.float64)[:, None]
    for m in (50, 3):  # the second call reuses the weight's table
        dy = synth.activations(g, m, 768)
        dx = UnifiedTensor.empty(ctx, [m, 512], DType.FP16)
        engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy, dtype=DType.FP16), w, dx, mfma=True)
        max_abs, rel, ok = f16_tol_check(dx.to_vec(), dy.astype(np.float64) @ truthw)
        assert ok, (m, max_abs, rel)


def test_dx_mfma_refusals(ctx, engine):
    import ctypes
    from rusty_amd import _lib
    L = _lib.lib()
    g = synth.rng(43)
    # affine codes, n_out not a multiple of 32: no table
    u, s, b = synth.affine_weight(g, 64, 128, group=64)
    wa = QuantizedTensor.affine(ctx, u, s, b, group=64)
    assert L.rq_qweight_dx_table_bytes(ctypes.byref(wa.descriptor())) == 0
    wr = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, 48, 64))
    assert L.rq_qweight_dx_table_bytes(ctypes.byref(wr.descriptor())) == 0
    with pytest.raises(ValueError):
        engine.qmatmul_dx(ctx, UnifiedTensor.empty(ctx, [2, 48]), wr, UnifiedTensor.empty(ctx, [2, 64]), mfma=True)
    w = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, 64, 64))
    d = w.descriptor()
    need = L.rq_qweight_dx_table_bytes(ctypes.byref(d))
    assert need >= 2 * 64 * 64 + 64 * 4
    table = UnifiedTensor.empty(ctx, [need], DType.U8)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qweight_dx_table", ctx.handle, ctypes.byref(d), table.ptr, need - 1, None)
    _lib.call("rq_qweight_dx_table", ctx.handle, ctypes.byref(d), table.ptr, need, None)
    dy = UnifiedTensor.new(ctx, np.ones((2, 64), np.float32))
    dx = UnifiedTensor.empty(ctx, [2, 64], DType.FP32)
    ws_need = L.rq_qmatmul_dx_mfma_workspace(2, 64)
    ws = UnifiedTensor.empty(ctx, [ws_need], DType.U8)
    with pytest.raises(RqError, match="RQ_ERR_INVALID_ARGUMENT"):
        _lib.call("rq_qmatmul_dx_mfma", ctx.handle, ctypes.byref(d), table.ptr, dy.ptr, 0, dx.ptr, 0, 2, ws.ptr,
                  ws_need - 1, None)
    _lib.call("rq_qmatmul_dx_mfma", ctx.handle, ctypes.byref(d), table.ptr, dy.ptr, 0, dx.ptr, 0, 2, ws.ptr,
              ws_need, None)
    ctx.sync()
