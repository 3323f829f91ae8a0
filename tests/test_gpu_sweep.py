"""Seeded sweeps over random shapes: the fused quantized linear (rq_qmatmul),
the SwiGLU MLP, and -- bit for bit -- the f32 matmul family and the
frozen-weight input gradient.  For the fused linear:

Forty cases drawn from one fixed seed: token counts across every dispatch tier
(the decode GEMVs at 1-2 tokens, the matrix-core GEMV at 3-16, the prefill
GEMM with and without split-K, the generic kernel where the fast ones refuse
a shape), ragged output counts, reduction lengths that are multiples of 64,
of 16 only, or odd, both weight formats (affine with its group straddling rows
where k_in % 64 != 0), and fp16 or f32 activations and outputs.  Each case is
checked on every output element against the oracle's f64 truth with the fp16
bar |dy| <= 2e-3*|y| + 2e-3*max|y| (f32 activations that a path casts to fp16
with a per-row power of two stay well inside it); shapes are sized so the
oracle finishes each in well under a second.
"""
import numpy as np
import pytest

from conftest import f16_tol_check
from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth

pytestmark = pytest.mark.gpu

F = {np.float16: DType.FP16, np.float32: DType.FP32}


def _cases(n_cases=40, seed=20261202):
    g = np.random.default_rng(seed)
    small = [1, 2, 3, 4, 5, 7, 8, 9, 12, 15, 16, 17, 24, 31, 33]
    large = [64, 100, 200, 300, 512]
    out = []
    while len(out) < n_cases:
        # every third case a prefill-sized token count
        m = int(g.choice(large if len(out) % 3 == 2 else small))
        kind = int(g.integers(0, 3))
        k = int(g.integers(1, 65)) * 64 if kind == 0 else (int(g.integers(1, 257)) * 16 if kind == 1
                                                             else int(g.integers(1, 2000)))
        n_max = min(3000, 60_000_000 // (m * k))
        if n_max < 1:
            continue
        n = int(g.integers(1, n_max + 1))
        fmt = int(g.integers(0, 2))
        xdt = np.float16 if g.integers(0, 2) else np.float32
        ydt = np.float16 if g.integers(0, 2) else np.float32
        out.append((m, n, k, fmt, xdt, ydt))
    return out


@pytest.mark.parametrize("m,n,k,fmt,xdt,ydt", _cases(),
                         ids=lambda v: v.__name__ if isinstance(v, type) else str(v))
def test_qmatmul_random_shapes(ctx, engine, m, n, k, fmt, xdt, ydt):
    g = synth.rng(m * 1_000_003 + n * 1009 + k + fmt)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n, k)
        b, w = None, QuantizedTensor.rowwise(ctx, q, s)
    else:
        q, s, b = synth.affine_weight(g, n, k, group=64)
        w = QuantizedTensor.affine(ctx, q, s, b, group=64)
    x = synth.activations(g, m, k, dtype=xdt)
    X = UnifiedTensor.new(ctx, x, dtype=F[xdt])
    Y = UnifiedTensor.new(ctx, np.full((m, n), np.nan, ydt), dtype=F[ydt])
    engine.qmatmul(ctx, X, w, Y)
    truth = orc.qlinear_truth(q, s, b, x.astype(np.float32), fmt)
    max_abs, rel, ok = f16_tol_check(Y.to_vec(), truth)
    print(f"[sweep m={m} n={n} k={k} fmt={fmt} x={np.dtype(xdt).name} y={np.dtype(ydt).name}] "
          f"max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert ok


def _mlp_cases(n_cases=12, seed=20261203):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        # every fourth case a prefill-sized token count
        m = int(g.choice([40, 200, 512] if len(out) % 4 == 3 else [1, 2, 3, 5, 8, 13, 16]))
        H = int(g.choice([64, 256, 1024, 2048, 4096, 1000]))
        i_max = min(3000, 90_000_000 // (3 * m * H))
        if i_max < 9:
            continue
        inter = int(g.integers(8, i_max + 1))
        xdt = np.float16 if g.integers(0, 2) else np.float32
        out.append((m, inter, H, xdt))
    return out


@pytest.mark.parametrize("m,inter,hidden,xdt", _mlp_cases(),
                         ids=lambda v: v.__name__ if isinstance(v, type) else str(v))
def test_swiglu_random_shapes(ctx, engine, m, inter, hidden, xdt):
    """The SwiGLU MLP (rq_mlp_swiglu) over random shapes, f32 output, against
    the oracle's f64 truth with h rounded to fp16 as the device stores it."""
    g = synth.rng(m * 7919 + inter * 31 + hidden)
    wg, sg = synth.rowwise_weight(g, inter, hidden)
    wu, su = synth.rowwise_weight(g, inter, hidden)
    wd, sd = synth.rowwise_weight(g, hidden, inter)
    x = synth.activations(g, m, hidden, dtype=xdt)
    Q = [QuantizedTensor.rowwise(ctx, a, b) for a, b in ((wg, sg), (wu, su), (wd, sd))]
    Y = UnifiedTensor.new(ctx, np.full((m, hidden), np.nan, np.float32), dtype=DType.FP32)
    engine.mlp_swiglu(ctx, UnifiedTensor.new(ctx, x, dtype=F[xdt]), *Q, Y)
    truth = orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32))
    max_abs, rel, ok = f16_tol_check(Y.to_vec(), truth)
    print(f"[sweep mlp m={m} I={inter} H={hidden} x={np.dtype(xdt).name}] max_abs={max_abs:.3e} rel={rel:.3e}",
          flush=True)
    assert ok


def _mm_cases(n_cases=16, seed=20261204):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        m, k, n = (int(v) for v in g.integers(1, [600, 1500, 900]))
        if m * k * n <= 30_000_000:
            out.append((m, k, n))
    return out


@pytest.mark.parametrize("m,k,n", _mm_cases())
def test_matmul_family_random_shapes_bit_exact(ctx, engine, m, k, n):
    """matmul / matmul_bt / matmul_at (kernels.wgsl:7-54, 234-252) over random
    shapes: bit for bit the oracle's k-ascending fused f32 loop."""
    g = np.random.default_rng(m * 31 + k * 7 + n)
    a = g.standard_normal((m, k), dtype=np.float32)
    b = g.standard_normal((k, n), dtype=np.float32)

    def run(op, x, y):
        out = UnifiedTensor.new(ctx, np.full((m, n), np.nan, np.float32))
        getattr(engine, op)(ctx, UnifiedTensor.new(ctx, x), UnifiedTensor.new(ctx, y), out)
        return out.to_vec().view(np.uint32)

    bt, at = np.ascontiguousarray(b.T), np.ascontiguousarray(a.T)
    assert np.array_equal(run("matmul", a, b), orc.matmul(a, b, fused=True).view(np.uint32))
    assert np.array_equal(run("matmul_bt", a, bt), orc.matmul_bt(a, bt, fused=True).view(np.uint32))
    assert np.array_equal(run("matmul_at", at, b), orc.matmul_at(at, b, fused=True).view(np.uint32))


def _dx_cases(n_cases=12, seed=20261205):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        m, n_out, k_in = (int(v) for v in g.integers(1, [300, 1500, 1500]))
        if m * n_out * k_in <= 40_000_000:
            out.append((m, n_out, k_in, int(g.integers(0, 2))))
    return out


@pytest.mark.parametrize("m,n_out,k_in,fmt", _dx_cases())
def test_dx_random_shapes_bit_exact(ctx, engine, m, n_out, k_in, fmt):
    """The frozen-weight input gradient (MatMulNode::backward's grad_a,
    rusty-autograd/src/lib.rs:152-158) over random shapes, f32: bit for bit the
    oracle's fused k-ascending matmul of dY with the dequantized weight."""
    g = synth.rng(m * 131 + n_out * 17 + k_in + fmt)
    if fmt == 0:
        q, s = synth.rowwise_weight(g, n_out, k_in)
        w, wdeq = QuantizedTensor.rowwise(ctx, q, s), orc.rowwise_dequantize(q, s)
    else:
        u, s, b = synth.affine_weight(g, n_out, k_in, group=64)
        w = QuantizedTensor.affine(ctx, u, s, b, group=64)
        wdeq = orc.affine_dequantize(u, s, b, group=64)
    dy = g.standard_normal((m, n_out), dtype=np.float32)
    dx = UnifiedTensor.new(ctx, np.full((m, k_in), np.nan, np.float32))
    engine.qmatmul_dx(ctx, UnifiedTensor.new(ctx, dy), w, dx)
    want = orc.matmul(dy, wdeq.reshape(n_out, k_in), fused=True)
    got = dx.to_vec()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))} elements differ"
