"""ctypes wrapper of ``oracle/liboracle.so`` -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed
CPU baseline), never as the product path.  See ``oracle.c`` for what each
function restates and how it is pinned.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_double, c_int, c_size_t, c_uint32, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = c_void_p
        L.orc_dequantize.argtypes = [P, c_size_t, P, c_size_t]
        L.orc_affine_dequantize.argtypes = [P, P, P, P, c_size_t, c_uint32, c_int]
        L.orc_rowwise_dequantize.argtypes = [P, P, P, c_size_t, c_size_t]
        for nm in ("orc_matmul", "orc_matmul_bt", "orc_matmul_at"):
            getattr(L, nm).argtypes = [P, P, P, c_int, c_int, c_int, c_int]
        L.orc_qlinear_truth.argtypes = [P, P, P, c_int, c_int, P, P, c_int, c_int, c_int]
        L.orc_ref_linear.argtypes = [P, P, P, c_int, c_int, P, P, P, c_int, c_int, c_int]
        L.orc_ref_linear.restype = c_int
        L.orc_ref_dequantize_linear.argtypes = [P, P, P, c_int, c_int, P, c_int, c_int]
        L.orc_ref_dequantize_linear.restype = c_int
        L.orc_ref_forward.argtypes = [P, P, P, c_int, c_int, c_int]
        L.orc_ref_forward.restype = c_int
        L.orc_swiglu_truth.argtypes = [P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int]
        L.orc_round_f16.argtypes = [c_double]
        L.orc_round_f16.restype = c_double
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def dequantize(words: np.ndarray, n_out: int) -> np.ndarray:
    """kernels.wgsl:153-166; elements past the written range stay NaN."""
    w = _c(words, np.uint32)
    out = np.full(n_out, np.nan, dtype=np.float32)
    lib().orc_dequantize(_p(w), w.size, _p(out), n_out)
    return out


def affine_dequantize(codes: np.ndarray, scales, biases, n: int | None = None, group: int = 64,
                      fused: bool = False) -> np.ndarray:
    """kernels.wgsl:379-400 over ``n`` elements (default: every code byte)."""
    b = _c(codes, np.uint8).ravel()
    n = b.size if n is None else n
    padded = np.zeros(-(-b.size // 4) * 4, dtype=np.uint8)
    padded[: b.size] = b
    s, bi = _c(scales, np.float32), _c(biases, np.float32)
    out = np.empty(n, dtype=np.float32)
    lib().orc_affine_dequantize(_p(padded), _p(s), _p(bi), _p(out), n, group, int(fused))
    return out


def rowwise_dequantize(q: np.ndarray, scales) -> np.ndarray:
    q = _c(q, np.int8)
    n, k = q.shape
    s = _c(scales, np.float32)
    out = np.empty((n, k), dtype=np.float32)
    lib().orc_rowwise_dequantize(_p(q), _p(s), _p(out), n, k)
    return out


def _mm(name, a, b, m, k, n, fused):
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty((m, n), dtype=np.float32)
    getattr(lib(), name)(_p(a), _p(b), _p(out), m, k, n, int(fused))
    return out


def matmul(a, b, fused=True):
    """kernels.wgsl:7-54: a [m,k] . b [k,n], k ascending."""
    m, k = a.shape
    return _mm("orc_matmul", a, b, m, k, b.shape[1], fused)


def matmul_bt(a, b, fused=True):
    """kernels.wgsl:234-242: a [m,k] . b[n,k]^T."""
    m, k = a.shape
    return _mm("orc_matmul_bt", a, b, m, k, b.shape[0], fused)


def matmul_at(a, b, fused=True):
    """kernels.wgsl:244-252: a[k,m]^T . b [k,n]."""
    k, m = a.shape
    return _mm("orc_matmul_at", a, b, m, k, b.shape[1], fused)


def qlinear_truth(codes, scales, biases, x, fmt: int, group: int = 64) -> np.ndarray:
    """f64 truth of Y = X . deq(W)^T; fmt 0 = signed per-row, 1 = affine u8."""
    codes = _c(codes, np.int8 if fmt == 0 else np.uint8)
    n, k = codes.shape
    x = _c(x, np.float32).reshape(-1, k)
    m = x.shape[0]
    s = _c(scales, np.float32)
    b = None if biases is None else _c(biases, np.float32)
    y = np.empty((m, n), dtype=np.float64)
    lib().orc_qlinear_truth(_p(codes), _p(s), _p(b), fmt, group, _p(x), _p(y), m, n, k)
    return y


def ref_linear(codes, scales, biases, x, fmt: int, group: int = 64):
    """The reference's path (dequantize -> f32 [in,out] -> k-ascending f32 GEMM).
    Returns (Y f32 [m, n], threads used)."""
    codes = _c(codes, np.int8 if fmt == 0 else np.uint8)
    n, k = codes.shape
    x = _c(x, np.float32).reshape(-1, k)
    m = x.shape[0]
    s = _c(scales, np.float32)
    b = None if biases is None else _c(biases, np.float32)
    y = np.empty((m, n), dtype=np.float32)
    wbuf = np.empty(n * k, dtype=np.float32)
    th = lib().orc_ref_linear(_p(codes), _p(s), _p(b), fmt, group, _p(x), _p(y), _p(wbuf), m, n, k)
    return y, th


class RefLinear:
    """The reference's Linear on CPU: f32 weight dequantized once at load
    (``orc_ref_dequantize_linear``), then ``forward`` per token."""

    def __init__(self, codes, scales, biases, fmt: int, group: int = 64):
        codes = _c(codes, np.int8 if fmt == 0 else np.uint8)
        self.n, self.k = codes.shape
        self.w = np.empty(self.n * self.k, dtype=np.float32)
        s = _c(scales, np.float32)
        b = None if biases is None else _c(biases, np.float32)
        lib().orc_ref_dequantize_linear(_p(codes), _p(s), _p(b), fmt, group, _p(self.w), self.n, self.k)

    def forward(self, x, out=None):
        x = _c(x, np.float32).reshape(-1, self.k)
        m = x.shape[0]
        y = np.empty((m, self.n), dtype=np.float32) if out is None else out
        threads = lib().orc_ref_forward(_p(self.w), _p(x), _p(y), m, self.n, self.k)
        return y, threads


def swiglu_truth(wg, sg, wu, su, wd, sd, x, h_round_f16=True):
    """rusty-graph/src/lib.rs:317-323 in f64: down(silu(gate x) * up x)."""
    wg, wu, wd = _c(wg, np.int8), _c(wu, np.int8), _c(wd, np.int8)
    inter, hidden = wg.shape
    x = _c(x, np.float32).reshape(-1, hidden)
    m = x.shape[0]
    y = np.empty((m, hidden), dtype=np.float64)
    hbuf = np.empty((m, inter), dtype=np.float64)
    lib().orc_swiglu_truth(_p(wg), _p(_c(sg, np.float32)), _p(wu), _p(_c(su, np.float32)), _p(wd),
                           _p(_c(sd, np.float32)), _p(x), _p(y), _p(hbuf), m, hidden, inter, int(h_round_f16))
    return y


def round_f16(v: float) -> float:
    return lib().orc_round_f16(v)
