"""MLX safetensors -> device weights -> kernels, against the oracle (GPU).

upload_dequantized must equal the oracle's affine dequantization bit for bit
(the reference's load-time result, kernels.wgsl:379-400) on the widened
scales/biases; upload_quantized must feed rq_qmatmul to the same tolerance as
any affine weight: |d| <= 2e-3*|y| + 2e-3*max|y| against the f64 truth.
"""
import numpy as np
import pytest

from conftest import f16_tol_check
from oracle import oracle as orc
from rusty_amd import DType, UnifiedTensor, synth
from rusty_amd.loader import QuantizationConfig, WeightsContext
from test_loader import mlx_file

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sdt,group", [("F16", 64), ("BF16", 32), ("F32", 128)])
def test_mlx_file_to_device(tmp_path, ctx, engine, sdt, group):
    g = synth.rng(group)
    n, k = 384, 1024
    codes = g.integers(0, 256, (n, k), dtype=np.uint8)
    s = g.uniform(0.001, 0.02, (n, k // group))
    b = -128 * s + g.uniform(-0.01, 0.01, (n, k // group))
    mlx_file(tmp_path / "model.safetensors", "model.layers.3.self_attn.o_proj", codes, s, b, sdt)
    wc = WeightsContext()
    wc.load_file(tmp_path / "model.safetensors")
    q = QuantizationConfig(group, 8, "affine")
    name = "model.layers.3.self_attn.o_proj"
    _, s32, b32 = wc._quantized_host(name, q)

    deq = wc.upload_dequantized(name, ctx, q)
    assert deq.shape == (n, k)  # logical shape, not the packed [n, k/4]
    want = orc.affine_dequantize(codes, s32, b32, group=group).reshape(n, k)
    assert np.array_equal(deq.to_vec().view(np.uint32), want.view(np.uint32))

    qt = wc.upload_quantized(name, ctx, q)
    for m in (1, 3, 80):
        x = synth.activations(g, m, k)
        y = UnifiedTensor.empty(ctx, [m, n], DType.FP32)
        engine.qmatmul(ctx, UnifiedTensor.new(ctx, x, dtype=DType.FP16), qt, y)
        truth = orc.qlinear_truth(codes, s32, b32, x.astype(np.float32), 1, group)
        max_abs, rel, ok = f16_tol_check(y.to_vec(), truth)
        print(f"[mlx {sdt} g{group} m={m}] max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
        assert ok
    wc.close()
