"""The device path against the committed golden fixtures (tests/golden/golden.npz).

Same bar as the other parity tests: dequantizers and the f32 matmul family
bit for bit; the fused linear and the SwiGLU MLP within the fp16 tolerance
|dy| <= 2e-3*|y| + 2e-3*max|y| of the frozen f64 truth.
"""
from pathlib import Path

import numpy as np
import pytest

from conftest import f16_tol_check
from rusty_amd import DType, QuantizedTensor, UnifiedTensor

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("case", [("dq_ka_words", "dq_ka_out"), ("dq_words", "dq_out")])
def test_dequantize(ctx, engine, gold, case):
    words, want = gold[case[0]], gold[case[1]]
    out = UnifiedTensor.new(ctx, np.full(want.size, -7.0, np.float32))
    engine.dequantize(ctx, UnifiedTensor.new(ctx, words, dtype=DType.U32), out)
    assert np.array_equal(bits(out.to_vec()), bits(want))


@pytest.mark.parametrize("case", [("af", 64, False, "af_out"), ("af", 64, True, "af_out_fma"),
                                  ("af32", 32, False, "af32_out")])
def test_affine_dequantize(ctx, engine, gold, case):
    p, group, fma, key = case
    u = gold[f"{p}_u"].ravel()
    codes = np.zeros(-(-u.size // 4) * 4, np.uint8)
    codes[: u.size] = u
    out = UnifiedTensor.new(ctx, np.full(u.size, np.nan, np.float32))
    engine.affine_dequantize(ctx, UnifiedTensor.new(ctx, codes.view(np.uint32), dtype=DType.U32),
                             UnifiedTensor.new(ctx, gold[f"{p}_s"]), UnifiedTensor.new(ctx, gold[f"{p}_b"]), out,
                             group=group, fma=fma)
    assert np.array_equal(bits(out.to_vec()), bits(gold[key]))


def test_rowwise_weight_dequantize(ctx, engine, gold):
    w = QuantizedTensor.rowwise(ctx, gold["rw_q"], gold["rw_s"])
    out = UnifiedTensor.empty(ctx, list(gold["rw_q"].shape))
    engine.dequantize_weight(ctx, w, out)
    assert np.array_equal(bits(out.to_vec()), bits(gold["rw_out"]))


@pytest.mark.parametrize("op,a,b,want", [("matmul", "mm_ka_a", None, "mm_ka_out"), ("matmul", "mm_a", "mm_b", "mm_out"),
                                         ("matmul_bt", "mm_a", "mmbt_b", "mmbt_out"),
                                         ("matmul_at", "mmat_a", "mm_b", "mmat_out")])
def test_matmul_family(ctx, engine, gold, op, a, b, want):
    A = gold[a]
    B = np.eye(2, dtype=np.float32) if b is None else gold[b]
    out = UnifiedTensor.new(ctx, np.full(gold[want].shape, np.nan, np.float32))
    getattr(engine, op)(ctx, UnifiedTensor.new(ctx, A), UnifiedTensor.new(ctx, B), out)
    assert np.array_equal(bits(out.to_vec()), bits(gold[want]))


@pytest.mark.parametrize("m", [3, 40])
@pytest.mark.parametrize("ydt", [np.float16, np.float32])
def test_qlinear_rowwise(ctx, engine, gold, m, ydt):
    w = QuantizedTensor.rowwise(ctx, gold["ql_q"], gold["ql_s"])
    X = UnifiedTensor.new(ctx, gold[f"ql_x{m}"], dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((m, 48), np.nan, ydt), dtype=DType.FP16 if ydt is np.float16 else DType.FP32)
    engine.qmatmul(ctx, X, w, Y)
    max_abs, rel, ok = f16_tol_check(Y.to_vec(), gold[f"ql_y{m}"])
    print(f"[golden qlinear m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def test_qlinear_affine(ctx, engine, gold):
    w = QuantizedTensor.affine(ctx, gold["qa_u"], gold["qa_s"], gold["qa_b"])
    X = UnifiedTensor.new(ctx, gold["qa_x"], dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((3, 48), np.nan, np.float32))
    engine.qmatmul(ctx, X, w, Y)
    assert f16_tol_check(Y.to_vec(), gold["qa_y"])[2]


def test_swiglu(ctx, engine, gold):
    G = QuantizedTensor.rowwise(ctx, gold["sw_wg"], gold["sw_sg"])
    U = QuantizedTensor.rowwise(ctx, gold["sw_wu"], gold["sw_su"])
    D = QuantizedTensor.rowwise(ctx, gold["sw_wd"], gold["sw_sd"])
    X = UnifiedTensor.new(ctx, gold["sw_x"], dtype=DType.FP16)
    Y = UnifiedTensor.new(ctx, np.full((2, 64), np.nan, np.float32))
    engine.mlp_swiglu(ctx, X, G, U, D, Y)
    assert f16_tol_check(Y.to_vec(), gold["sw_y"])[2]
