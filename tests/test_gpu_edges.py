"""Degenerate shapes through the C ABI on the device.

* no tokens (m = 0) or no output features (n_out = 0): the call succeeds and
  writes nothing (outputs keep their NaN fill);
* an empty reduction (k_in = 0, and for the SwiGLU MLP no intermediate
  features): every output is the empty sum, 0, for both weight formats and
  both output dtypes, from one token to a prefill-sized batch.

The reference's matmul over an empty k stores 0 (`kernels.wgsl:7-54`: the
accumulator starts at 0 and the k loop runs no step); its Linear over empty
inputs returns an empty tensor.
"""
import ctypes

import numpy as np
import pytest

from rusty_amd import DType, QuantizedTensor, UnifiedTensor, _lib, synth

pytestmark = pytest.mark.gpu

F = {np.float16: DType.FP16, np.float32: DType.FP32}


def weight(ctx, g, fmt, n, k):
    if fmt == "rowwise":
        return QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, n, k))
    u, s, b = synth.affine_weight(g, n, k, group=64)
    if s.size == 0:  # an empty weight still carries its (unused) scale array
        s, b = np.ones(1, np.float32), np.zeros(1, np.float32)
    return QuantizedTensor.affine(ctx, u, s, b, group=64)


def nan_out(ctx, m, n, ydt):
    return UnifiedTensor.new(ctx, np.full((m, n), np.nan, ydt), dtype=F[ydt])


@pytest.mark.parametrize("m", [1, 2, 5, 16, 300])
@pytest.mark.parametrize("fmt", ["rowwise", "affine"])
@pytest.mark.parametrize("ydt", [np.float16, np.float32])
def test_qmatmul_empty_reduction_is_zero(ctx, engine, m, fmt, ydt):
    g = synth.rng(m)
    w = weight(ctx, g, fmt, 96, 0)
    y = nan_out(ctx, m, 96, ydt)
    d = w.descriptor()
    # no activation bytes exist: a null x is accepted
    _lib.call("rq_qmatmul", ctx.handle, ctypes.byref(d), None, _lib.RQ_F16, y.ptr,
              _lib.RQ_F32 if ydt == np.float32 else _lib.RQ_F16, m, None)
    got = y.to_vec()
    assert not np.isnan(got).any() and not got.any()


@pytest.mark.parametrize("m,n", [(0, 64), (3, 0), (0, 0)])
def test_qmatmul_nothing_to_write(ctx, engine, m, n):
    g = synth.rng(7)
    w = QuantizedTensor.rowwise(ctx, *synth.rowwise_weight(g, n, 64))
    x = UnifiedTensor.new(ctx, synth.activations(g, max(m, 1), 64), dtype=DType.FP16)
    sentinel = nan_out(ctx, 4, 4, np.float32)
    d = w.descriptor()
    _lib.call("rq_qmatmul", ctx.handle, ctypes.byref(d), x.ptr, _lib.RQ_F16, sentinel.ptr, _lib.RQ_F32, m, None)
    assert np.isnan(sentinel.to_vec()).all()


@pytest.mark.parametrize("m", [1, 4, 40])
@pytest.mark.parametrize("noalloc", [False, True])
def test_swiglu_without_intermediate_features_is_zero(ctx, engine, m, noalloc):
    """gate/up [0, H], down [H, 0]: h is empty and y = down . h = 0."""
    g = synth.rng(11)
    H = 128
    gate, up = (QuantizedTensor.rowwise(ctx, np.zeros((0, H), np.int8), np.zeros(0, np.float32)) for _ in range(2))
    down = QuantizedTensor.rowwise(ctx, np.zeros((H, 0), np.int8), g.uniform(0.001, 0.02, H).astype(np.float32))
    x = UnifiedTensor.new(ctx, synth.activations(g, m, H), dtype=DType.FP16)
    y = nan_out(ctx, m, H, np.float32)
    dg, du, dd = gate.descriptor(), up.descriptor(), down.descriptor()
    if noalloc:
        _lib.call("rq_mlp_swiglu_noalloc", ctx.handle, ctypes.byref(dg), ctypes.byref(du), ctypes.byref(dd), x.ptr,
                  _lib.RQ_F16, y.ptr, _lib.RQ_F32, m, None)
    else:
        # an empty workspace: h may be null
        _lib.call("rq_mlp_swiglu", ctx.handle, ctypes.byref(dg), ctypes.byref(du), ctypes.byref(dd), x.ptr,
                  _lib.RQ_F16, None, y.ptr, _lib.RQ_F32, m, None)
    got = y.to_vec()
    assert not np.isnan(got).any() and not got.any()


@pytest.mark.parametrize("tree", [False, True])
@pytest.mark.parametrize("m", [1, 300])
def test_lora_empty_reduction_is_zero(ctx, engine, tree, m):
    """k_in = 0 with a rank-4 adapter: x . A is empty (0), so y = 0 + 0 . B."""
    g = synth.rng(12)
    n, rank = 80, 4
    w = QuantizedTensor.rowwise(ctx, np.zeros((n, 0), np.int8), g.uniform(0.001, 0.02, n).astype(np.float32))
    b = UnifiedTensor.new(ctx, g.standard_normal((rank, n), dtype=np.float32))
    a = UnifiedTensor.empty(ctx, [0, rank], DType.FP32)
    y = nan_out(ctx, m, n, np.float32)
    flags = _lib.RQ_LORA_TREE if tree else 0
    need = _lib.lib().rq_qmatmul_lora_ex_workspace(m, 0, n, rank, _lib.RQ_F16, _lib.RQ_F32, flags)
    ws = UnifiedTensor.empty(ctx, [max(need, 1)], DType.U8)
    d = w.descriptor()
    _lib.call("rq_qmatmul_lora_ex", ctx.handle, ctypes.byref(d), None, _lib.RQ_F16, a.ptr or None, b.ptr, rank,
              y.ptr, _lib.RQ_F32, m, flags, ws.ptr, max(need, 1), None)
    got = y.to_vec()
    assert not np.isnan(got).any() and not got.any()


@pytest.mark.parametrize("fmt", ["rowwise", "affine"])
def test_dx_without_output_features_is_zero(ctx, engine, fmt):
    """n_out = 0: dX = dY . deq(W) sums over no output feature."""
    g = synth.rng(13)
    m, k = 5, 96
    if fmt == "rowwise":
        w = QuantizedTensor.rowwise(ctx, np.zeros((0, k), np.int8), np.zeros(0, np.float32))
    else:
        w = QuantizedTensor.affine(ctx, np.zeros((0, k), np.uint8), np.ones(1, np.float32), np.zeros(1, np.float32),
                                   group=64)
    dx = nan_out(ctx, m, k, np.float32)
    d = w.descriptor()
    _lib.call("rq_qmatmul_dx", ctx.handle, ctypes.byref(d), None, _lib.RQ_F32, dx.ptr, _lib.RQ_F32, m, None)
    got = dx.to_vec()
    assert not np.isnan(got).any() and not got.any()
