"""Measurement aids and memory plumbing of the C ABI: rq_device_delay (the
bounded device-side wait that benchmark drivers put in front of a batch of
direct launches), rq_stream_probe (the GEMV's weight stream alone) and
rq_fma_chain_probe (one wave's dependent fma chain), none with a reference
counterpart, and rq_memset."""
import pytest

from rusty_amd import _lib
from rusty_amd.hiprt import Event

pytestmark = pytest.mark.gpu


def test_device_delay_holds_the_stream(ctx):
    a, b = Event(), Event()
    a.record(ctx.stream)
    _lib.call("rq_device_delay", ctx.handle, 2000, None)
    b.record(ctx.stream)
    b.synchronize()
    ms = a.elapsed_ms(b)
    assert 1.9 <= ms <= 50.0, ms


def test_device_delay_limits(ctx):
    lib = _lib.lib()
    assert lib.rq_device_delay(ctx.handle, 0, None) == _lib.RQ_OK
    assert lib.rq_device_delay(ctx.handle, 100001, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert b"100000" in lib.rq_last_error()
    ctx.sync()


# rq_memset: a fill kernel, exact for any alignment and length, and safe to
# capture in a HIP graph (replayed several times with eager writes between)

@pytest.mark.parametrize("offset,nbytes", [(0, 0), (0, 1), (3, 5), (1, 16), (7, 33), (0, 4096), (5, 100003)])
def test_memset_bytes(ctx, offset, nbytes):
    import numpy as np

    from rusty_amd import DType, UnifiedTensor

    total = offset + nbytes + 37
    buf = UnifiedTensor.new(ctx, np.full(total, 0xAB, np.uint8), dtype=DType.U8)
    _lib.call("rq_memset", ctx.handle, buf.ptr + offset, 0x5C, nbytes, None)
    got = buf.to_vec()
    want = np.full(total, 0xAB, np.uint8)
    want[offset:offset + nbytes] = 0x5C
    assert np.array_equal(got, want)


def test_memset_in_graph_replays(ctx):
    import numpy as np

    from rusty_amd import DType, UnifiedTensor
    from rusty_amd.hiprt import Graph

    n = 1 << 20
    buf = UnifiedTensor.new(ctx, np.full(n + 9, 7, np.uint8), dtype=DType.U8)
    g = Graph(ctx.stream, lambda: _lib.call("rq_memset", ctx.handle, buf.ptr + 3, 0, n, None))
    ones = np.full(n + 9, 0xFF, np.uint8)
    for _ in range(4):
        _lib.call("rq_memcpy_h2d", ctx.handle, buf.ptr, ones.ctypes.data, n + 9, None)  # eager write between replays
        g.launch()
        ctx.sync()
        got = buf.to_vec()
        assert (got[3:3 + n] == 0).all() and (got[:3] == 0xFF).all() and (got[3 + n:] == 0xFF).all()


# The hot path captured once in a HIP graph and replayed with new activations
# written (eagerly) between replays: every replay must match the oracle.

@pytest.mark.parametrize("m", [1, 8, 300])
def test_qmatmul_graph_replays(ctx, engine, m):
    import numpy as np

    from conftest import f16_tol_check
    from oracle import oracle as orc
    from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth
    from rusty_amd.hiprt import Graph

    g = synth.rng(900 + m)
    q, s = synth.rowwise_weight(g, 520, 1024)
    w = QuantizedTensor.rowwise(ctx, q, s)
    X = UnifiedTensor.empty(ctx, [m, 1024], DType.FP16)
    Y = UnifiedTensor.empty(ctx, [m, 520], DType.FP16)
    graph = Graph(ctx.stream, lambda: engine.qmatmul(ctx, X, w, Y))
    for rep in range(3):
        x = synth.activations(g, m, 1024)
        _lib.call("rq_memcpy_h2d", ctx.handle, X.ptr, x.ctypes.data, x.nbytes, None)
        graph.launch()
        ctx.sync()
        _, _, ok = f16_tol_check(Y.to_vec(), orc.qlinear_truth(q, s, None, x.astype(np.float32), 0))
        assert ok, f"replay {rep}"


def test_swiglu_graph_replays(ctx, engine):
    import numpy as np

    from conftest import f16_tol_check
    from oracle import oracle as orc
    from rusty_amd import DType, QuantizedTensor, UnifiedTensor, synth
    from rusty_amd.hiprt import Graph

    g = synth.rng(950)
    wg, sg = synth.rowwise_weight(g, 384, 512)
    wu, su = synth.rowwise_weight(g, 384, 512)
    wd, sd = synth.rowwise_weight(g, 512, 384)
    G, U, D = (QuantizedTensor.rowwise(ctx, a, b) for a, b in ((wg, sg), (wu, su), (wd, sd)))
    for m in (1, 4):
        X = UnifiedTensor.empty(ctx, [m, 512], DType.FP16)
        Y = UnifiedTensor.empty(ctx, [m, 512], DType.FP32)
        H = UnifiedTensor.empty(ctx, [2, m, 384], DType.FP16)
        graph = Graph(ctx.stream, lambda: engine.mlp_swiglu(ctx, X, G, U, D, Y, H))
        for rep in range(3):
            x = synth.activations(g, m, 512)
            _lib.call("rq_memcpy_h2d", ctx.handle, X.ptr, x.ctypes.data, x.nbytes, None)
            graph.launch()
            ctx.sync()
            truth = orc.swiglu_truth(wg, sg, wu, su, wd, sd, x.astype(np.float32))
            assert f16_tol_check(Y.to_vec(), truth)[2], f"m={m} replay {rep}"


# rq_stream_probe: the GEMV's weight stream without arithmetic (a measurement
# aid, no reference counterpart).  Wave w of block b XOR-combines the 16-byte
# chunks its 64 lanes loaded (chunks 64w .. 64w + 63, + 256 j) over the
# block's rows; with store, lane 0 writes it, folded to 16 bits, for row b*R + w.

def _probe_expect(src, row_bytes, rows, R):
    import numpy as np

    words = src.view(np.uint32).reshape(rows, row_bytes // 4)
    out = np.zeros(rows, np.uint16)
    C = row_bytes // 16
    for b in range(-(-rows // R)):
        here = min(R, rows - b * R)
        for w in range(here):
            chunks = [c for c0 in range(64 * w, C, 256) for c in range(c0, min(c0 + 64, C))]
            acc = 0
            for r in range(here):
                for c in chunks:
                    for v in words[b * R + r, 4 * c:4 * c + 4]:
                        acc ^= int(v)
            out[b * R + w] = (acc ^ (acc >> 16)) & 0xFFFF
    return out


@pytest.mark.parametrize("row_bytes,rows,R", [(4096, 10, 4), (8192, 7, 2), (16384, 3, 1), (2048, 5, 3)])
def test_stream_probe_store(ctx, row_bytes, rows, R):
    import numpy as np

    from rusty_amd import DType, UnifiedTensor

    src = np.random.default_rng(row_bytes + rows).integers(0, 256, rows * row_bytes, dtype=np.uint8)
    s = UnifiedTensor.new(ctx, src, dtype=DType.U8)
    d = UnifiedTensor.new(ctx, np.full(rows + 8, 0xDEAD, np.uint16).view(np.uint8), dtype=DType.U8)
    # store == 0: the loads are consumed, nothing is written
    _lib.call("rq_stream_probe", ctx.handle, s.ptr, row_bytes, rows, R, d.ptr, 0, None)
    assert np.all(d.to_vec().view(np.uint16) == 0xDEAD)
    _lib.call("rq_stream_probe", ctx.handle, s.ptr, row_bytes, rows, R, d.ptr, 1, None)
    got = d.to_vec().view(np.uint16)
    np.testing.assert_array_equal(got[:rows], _probe_expect(src, row_bytes, rows, R))
    assert np.all(got[rows:] == 0xDEAD)  # nothing past the rows


def test_stream_probe_limits(ctx):
    lib = _lib.lib()
    assert lib.rq_stream_probe(ctx.handle, None, 16, 1, 1, 16, 1, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_stream_probe(ctx.handle, 16, 16, 1, 1, None, 1, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_stream_probe(ctx.handle, 16, 24, 1, 1, 16, 1, None) == _lib.RQ_ERR_SHAPE
    assert lib.rq_stream_probe(ctx.handle, 16, 16, 1, 5, 16, 1, None) == _lib.RQ_ERR_SHAPE
    assert lib.rq_stream_probe(ctx.handle, 16, 16384 + 16, 1, 1, 16, 1, None) == _lib.RQ_ERR_SHAPE


# rq_fma_chain_probe: lane l of one wave runs acc = fma(acc, a, b) from acc = l,
# a = 1.0000001f, b = 1e-7f; checked against the C library's fmaf (one rounding).

@pytest.mark.parametrize("steps", [0, 1, 37, 1000])
def test_fma_chain_probe(ctx, steps):
    import ctypes

    import numpy as np

    from rusty_amd import DType, UnifiedTensor

    libm = ctypes.CDLL("libm.so.6")
    libm.fmaf.restype = ctypes.c_float
    libm.fmaf.argtypes = [ctypes.c_float] * 3
    a, b = float(np.float32(1.0000001)), float(np.float32(1e-7))
    want = np.zeros(64, np.float32)
    for lane in range(64):
        acc = float(lane)
        for _ in range(steps):
            acc = libm.fmaf(acc, a, b)
        want[lane] = acc
    d = UnifiedTensor.new(ctx, np.full(64, np.nan, np.float32))
    _lib.call("rq_fma_chain_probe", ctx.handle, steps, d.ptr, None)
    np.testing.assert_array_equal(d.to_vec(), want)


def test_fma_chain_probe_limits(ctx):
    lib = _lib.lib()
    assert lib.rq_fma_chain_probe(ctx.handle, 10, None, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_fma_chain_probe(ctx.handle, -1, 16, None) == _lib.RQ_ERR_SHAPE


# rq_device_clock: device wall-clock stamps on the stream (graph-capturable)

def test_device_clock_brackets_a_delay(ctx):
    import ctypes

    import numpy as np

    from rusty_amd import DType, UnifiedTensor

    buf = UnifiedTensor.new(ctx, np.zeros(16, np.uint8), dtype=DType.U8)
    hz = ctypes.c_uint64()
    _lib.call("rq_device_clock", ctx.handle, buf.ptr, ctypes.byref(hz), None)
    _lib.call("rq_device_delay", ctx.handle, 3000, None)
    _lib.call("rq_device_clock", ctx.handle, buf.ptr + 8, None, None)
    t = buf.to_vec().view(np.uint64)
    ms = (int(t[1]) - int(t[0])) / hz.value * 1e3
    assert 1e6 <= hz.value <= 1e10
    assert 2.9 <= ms <= 50.0, ms
    assert _lib.lib().rq_device_clock(ctx.handle, None, None, None) == _lib.RQ_ERR_INVALID_ARGUMENT
