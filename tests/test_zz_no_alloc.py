"""GPU check of rq_mlp_swiglu_noalloc, the SwiGLU MLP whose intermediate lives
in the library's per-device scratch array instead of a caller workspace.

Called through the C ABI and compared with rq_mlp_swiglu on the same inputs:
the two run the same kernels, so y must agree bit for bit.  Two calls in a
row, the second with fewer tokens (the array keeps the first call's h), for
the decode (m <= 16) and prefill (m > 16) paths; sizes past the array are
refused with RQ_ERR_SHAPE before anything is launched.
"""
import ctypes

import numpy as np
import pytest

from rusty_amd import DType, QuantizedTensor, RqError, UnifiedTensor, _lib, synth

pytestmark = pytest.mark.gpu


def _weights(ctx, g, inter, hidden):
    G = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, inter, hidden))
    U = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, inter, hidden))
    D = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, hidden, inter))
    return G, U, D


def _noalloc(ctx, x, G, U, D, ydt):
    m = x.shape[0]
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((m, D.n_out), np.nan, ydt), dtype=DType.FP32 if ydt is np.float32 else DType.FP16)
    dg, du, dd = G.descriptor(), U.descriptor(), D.descriptor()
    _lib.call("rq_mlp_swiglu_noalloc", ctx.handle, ctypes.byref(dg), ctypes.byref(du), ctypes.byref(dd), X.ptr,
              _lib.RQ_F16, Y.ptr, _lib.RQ_F32 if ydt is np.float32 else _lib.RQ_F16, m, None)
    return Y.to_vec()


def _with_workspace(ctx, engine, x, G, U, D, ydt):
    X = UnifiedTensor.new(ctx, x, dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((x.shape[0], D.n_out), np.nan, ydt),
                          dtype=DType.FP32 if ydt is np.float32 else DType.FP16)
    engine.mlp_swiglu(ctx, X, G, U, D, Y)
    return Y.to_vec()


@pytest.mark.parametrize("m1,m2,inter,hidden", [(16, 3, 1376, 1024), (1, 1, 2048, 512), (64, 24, 768, 512)],
                         ids=["decode_16_then_3", "decode_1_then_1", "prefill_64_then_24"])
def test_noalloc_matches_workspace_variant(ctx, engine, m1, m2, inter, hidden):
    g = synth.rng(900 + m1 + inter)
    G, U, D = _weights(ctx, g, inter, hidden)
    for m in (m1, m2):  # second call smaller: the scratch still holds the first call's h
        x = synth.activations(g, m, hidden)
        ref = _with_workspace(ctx, engine, x, G, U, D, np.float32)
        got = _noalloc(ctx, x, G, U, D, np.float32)
        assert np.isfinite(ref).all()
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
        print(f"[noalloc m={m} I={inter} H={hidden}] bit-exact vs rq_mlp_swiglu", flush=True)


def test_noalloc_refuses_sizes_past_the_scratch(ctx):
    g = synth.rng(950)
    inter, hidden = 1024, 256
    G, U, D = _weights(ctx, g, inter, hidden)
    m = 2049  # 4 * m * inter bytes > 8 MiB
    X = UnifiedTensor.new(ctx, synth.activations(g, m, hidden), dtype=DType.FP16)
    Y = UnifiedTensor.empty(ctx, [m, hidden], DType.FP32)
    dg, du, dd = G.descriptor(), U.descriptor(), D.descriptor()
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        _lib.call("rq_mlp_swiglu_noalloc", ctx.handle, ctypes.byref(dg), ctypes.byref(du), ctypes.byref(dd), X.ptr,
                  _lib.RQ_F16, Y.ptr, _lib.RQ_F32, m, None)
    # the largest size that fits still runs
    m = 2048
    x = synth.activations(g, m, hidden)
    ok = _noalloc(ctx, x, G, U, D, np.float32)
    assert np.isfinite(ok).all()
