"""GPU parity of the standalone dequantizers against the CPU oracle, bit-exact.

rq_dequantize          <- kernels.wgsl:153-166 / lib.rs:4872-4899
rq_affine_dequantize   <- kernels.wgsl:379-400 / lib.rs:4939-4990 (both roundings)
rq_qweight_dequantize     load-time dequantization of a weight (both formats)
"""
import numpy as np
import pytest

from oracle import oracle as orc
from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_dequantize_known_answer(ctx, engine):
    # rusty-loader/examples/load_and_run.rs:18-34 through the device path
    inp = UnifiedTensor.new(ctx, np.array([1.0, 2.0, 3.0, 4.0], np.float32), [4])
    out = UnifiedTensor.empty(ctx, [4])
    engine.dequantize(ctx, inp, out)
    assert out.to_vec().tolist() == [0.0, 0.0, 128.0, 63.0]


@pytest.mark.parametrize("n_words,n_out", [(1, 4), (5, 17), (5, 20), (64, 200), (1000, 4003), (262144, 1 << 20)])
def test_dequantize_matches_oracle(ctx, engine, n_words, n_out):
    g = np.random.default_rng(n_words)
    words = g.integers(0, 2**32, n_words, dtype=np.uint32)
    inp = UnifiedTensor.new(ctx, words, dtype=DType.U32)
    sentinel = np.full(n_out, -7.0, np.float32)
    out = UnifiedTensor.new(ctx, sentinel)
    engine.dequantize(ctx, inp, out)
    got = out.to_vec()
    want = orc.dequantize(words, n_out)
    written = min(4 * n_words, n_out)
    assert np.array_equal(bits(got[:written]), bits(want[:written]))
    assert np.all(got[written:] == -7.0), "elements past the data must stay untouched"


AFFINE_SHAPES = [
    (64, 1024),        # C1-sized rows, one group per 64
    (7, 100),          # n % 64 != 0, n % 16 != 0, n % 4 == 0
    (3, 33),           # n % 4 != 0: byte tail
    (4096, 4096),      # 16.7M elements: beyond the reference's 4,194,240 coverage cap
]


@pytest.mark.parametrize("fma", [False, True])
@pytest.mark.parametrize("shape", AFFINE_SHAPES)
def test_affine_dequantize_bit_exact(ctx, engine, shape, fma):
    n_rows, k = shape
    g = synth.rng(sum(shape))
    u, s, b = synth.affine_weight(g, n_rows, k)
    n = n_rows * k
    codes = np.zeros(-(-n // 4) * 4, np.uint8)
    codes[:n] = u.ravel()
    w = UnifiedTensor.new(ctx, codes.view(np.uint32), dtype=DType.U32)
    st, bt = UnifiedTensor.new(ctx, s), UnifiedTensor.new(ctx, b)
    out = UnifiedTensor.empty(ctx, [n])
    engine.affine_dequantize(ctx, w, st, bt, out, fma=fma)
    got = out.to_vec()
    want = orc.affine_dequantize(u, s, b, fused=fma)
    assert np.array_equal(bits(got), bits(want)), f"{np.count_nonzero(bits(got) != bits(want))} elements differ"


def test_affine_group_sizes_and_unaligned(ctx, engine):
    g = synth.rng(77)
    for group in (16, 32, 128, 5):
        u, s, b = synth.affine_weight(g, 9, 160, group=group)
        n = u.size
        w = UnifiedTensor.new(ctx, u.ravel(), dtype=DType.U8)
        out = UnifiedTensor.empty(ctx, [n + 1])
        # unaligned output: write into out+1 element (4-byte aligned, not 16)
        view = UnifiedTensor(ctx, out.ptr + 4, [n], DType.FP32, owner=False)
        engine.affine_dequantize(ctx, w, UnifiedTensor.new(ctx, s), UnifiedTensor.new(ctx, b), view, group=group)
        got = out.to_vec()[1:]
        assert np.array_equal(bits(got), bits(orc.affine_dequantize(u, s, b, group=group))), group


@pytest.mark.parametrize("group", [16, 32, 48, 128])
def test_affine_group_sizes_aligned(ctx, engine, group):
    """Aligned pointers take the wave-step path (1024 elements per wave step,
    each lane's 4-element pieces 256 apart): a power-of-two group by shift, 48
    by division; 9 x 480 elements = 4 full steps + a 224-element tail."""
    g = synth.rng(300 + group)
    u, s, b = synth.affine_weight(g, 9, 480, group=group)
    w = UnifiedTensor.new(ctx, u.ravel(), dtype=DType.U8)
    out = UnifiedTensor.empty(ctx, [u.size])
    engine.affine_dequantize(ctx, w, UnifiedTensor.new(ctx, s), UnifiedTensor.new(ctx, b), out, group=group)
    assert np.array_equal(bits(out.to_vec()), bits(orc.affine_dequantize(u, s, b, group=group))), group


@pytest.mark.parametrize("shape", [(1024, 1024), (4096, 4096), (11008, 4096), (5, 24), (3, 7), (3, 1040)])
def test_rowwise_weight_dequantize_bit_exact(ctx, engine, shape):
    g = synth.rng(shape[0])
    q, s = synth.rowwise_weight(g, *shape)
    w = QuantizedTensor.rowwise(ctx, q, s)
    out = UnifiedTensor.empty(ctx, list(shape))
    engine.dequantize_weight(ctx, w, out)
    assert np.array_equal(bits(out.to_vec()), bits(orc.rowwise_dequantize(q, s)))


def test_affine_weight_dequantize_bit_exact(ctx, engine):
    g = synth.rng(5)
    u, s, b = synth.affine_weight(g, 1024, 1024)
    w = QuantizedTensor.affine(ctx, u, s, b)
    out = UnifiedTensor.empty(ctx, [1024, 1024])
    engine.dequantize_weight(ctx, w, out)
    assert np.array_equal(bits(out.to_vec().ravel()), bits(orc.affine_dequantize(u, s, b)))


def test_affine_shape_errors(ctx, engine):
    from rusty_amd import RqError

    w = UnifiedTensor.new(ctx, np.zeros(4, np.uint32), dtype=DType.U32)
    s = UnifiedTensor.new(ctx, np.ones(1, np.float32))
    out = UnifiedTensor.empty(ctx, [128])  # needs 32 words and 2 groups
    with pytest.raises(RqError, match="RQ_ERR_SHAPE"):
        engine.affine_dequantize(ctx, w, s, s, out)
