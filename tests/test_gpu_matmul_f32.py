"""GPU parity of the f32 matmul family against the oracle, bit-exact.

rq_matmul    <- kernels.wgsl:7-54    (matmul_tiled)  / lib.rs:4403-4453
rq_matmul_bt <- kernels.wgsl:234-242 (matmul_bt)     / lib.rs:4299-4349
rq_matmul_at <- kernels.wgsl:244-252 (matmul_at)     / lib.rs:4351-4401

The device keeps one f32 accumulator per output updated in ascending k with
fma, so it must equal the oracle's fused k-ascending loop bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from rusty_amd import UnifiedTensor

pytestmark = pytest.mark.gpu

# Few outputs or few 64x64 tiles take the one-output-per-thread chain kernel
# (k-chunks of 256 or 512 staged in LDS, column tiles of 8/16/32/64): k past
# a chunk and not a multiple of 32, k = 0, every column-tile width; the others
# (512x200x520, 1030x64x600) the 64x64 tiled kernel.  Both must match the
# oracle bit for bit.
SHAPES = [(2, 2, 2), (1, 1024, 1024), (8, 1024, 1024), (65, 33, 70), (128, 256, 96), (3, 0, 5), (1, 4096, 4096),
          (1, 4097, 16), (5, 1000, 40), (33, 600, 9), (7, 300, 3), (2, 513, 100), (512, 4096, 16),
          (512, 200, 520), (1030, 64, 600),
          # the DMA-ring chain kernel (16-byte rows, n > 16 or A.B^T): ragged row and
          # column blocks with a partial last chunk, for all three variants
          (20, 520, 44), (12, 700, 36)]


def _run(engine, ctx, op, a, b, m, n):
    A, B = UnifiedTensor.new(ctx, a), UnifiedTensor.new(ctx, b)
    out = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
    getattr(engine, op)(ctx, A, B, out)
    return out.to_vec()


def test_identity_known_answer(ctx, engine):
    # rusty-backend/examples/ops_test.rs:13-17
    got = _run(engine, ctx, "matmul", np.array([[1, 2], [3, 4]], np.float32), np.eye(2, dtype=np.float32), 2, 2)
    assert got.ravel().tolist() == [1, 2, 3, 4]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_family_bit_exact(ctx, engine, m, k, n):
    g = np.random.default_rng(m * 7 + k + n)
    a = g.standard_normal((m, k), dtype=np.float32)
    b = g.standard_normal((k, n), dtype=np.float32)
    want = orc.matmul(a, b, fused=True)
    assert np.array_equal(_run(engine, ctx, "matmul", a, b, m, n).view(np.uint32), want.view(np.uint32))
    bt = np.ascontiguousarray(b.T)
    assert np.array_equal(_run(engine, ctx, "matmul_bt", a, bt, m, n).view(np.uint32),
                          orc.matmul_bt(a, bt, fused=True).view(np.uint32))
    at = np.ascontiguousarray(a.T)
    assert np.array_equal(_run(engine, ctx, "matmul_at", at, b, m, n).view(np.uint32),
                          orc.matmul_at(at, b, fused=True).view(np.uint32))


def test_k_ascending_order(ctx, engine):
    a = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    assert _run(engine, ctx, "matmul", a, np.ones((4, 1), np.float32), 1, 1).item() == 1.0


def test_shape_mismatch_raises(ctx, engine):
    A = UnifiedTensor.new(ctx, np.zeros((2, 3), np.float32))
    B = UnifiedTensor.new(ctx, np.zeros((4, 5), np.float32))
    out = UnifiedTensor.empty(ctx, [2, 5])
    with pytest.raises(ValueError):
        engine.matmul(ctx, A, B, out)
