"""Host-side mirror of Rusty's backend op surface over the gfx950 C ABI.

Names and argument meaning follow the reference so code written against
``rusty_backend`` reads the same here:

==============================  ==================================================
reference (rusty-backend)        here
==============================  ==================================================
``WgpuContext::new``  lib.rs:20  :class:`WgpuContext` (device, own HIP stream)
``UnifiedTensor``  lib.rs:79     :class:`UnifiedTensor` (device buffer + shape)
``ComputeEngine::new`` lib.rs:343 :class:`ComputeEngine`
``dequantize``  lib.rs:4872      :meth:`ComputeEngine.dequantize`
``affine_dequantize`` lib.rs:4939 :meth:`ComputeEngine.affine_dequantize`
``matmul``  lib.rs:4403          :meth:`ComputeEngine.matmul`
``matmul_bt``  lib.rs:4299       :meth:`ComputeEngine.matmul_bt`
``matmul_at``  lib.rs:4351       :meth:`ComputeEngine.matmul_at`
(none: weights are f32)          :class:`QuantizedTensor`, :meth:`ComputeEngine.qmatmul`
==============================  ==================================================

As in the reference, ops are enqueued asynchronously on the context's stream
and ``to_vec`` waits for them.  Unlike the reference, a wrong shape raises
:class:`rusty_amd._lib.RqError` instead of reading clamped memory.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import call, rq_qweight


class DType(enum.Enum):
    """Element type of a device buffer.  FP32/FP16 are the reference's
    ``DType`` (lib.rs:57-76); the byte types carry quantized codes and packed
    words, which the reference passes as raw ``wgpu::Buffer``s."""

    FP32 = np.float32
    FP16 = np.float16
    I8 = np.int8
    U8 = np.uint8
    U32 = np.uint32

    @property
    def np(self):
        return np.dtype(self.value)

    @property
    def itemsize(self) -> int:
        return self.np.itemsize


def _prod(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


class WgpuContext:
    """Device context (replaces ``WgpuContext::new``, lib.rs:20-47).

    Kept under the reference's name so callers port unchanged; it owns a HIP
    context on a gfx950 device, not a wgpu adapter."""

    def __init__(self, device: int = 0):
        lib = _lib.lib()
        h = ctypes.c_void_p()
        call("rq_ctx_create", device, ctypes.byref(h))
        self._h = h
        self._lib = lib
        self.device = device
        s = ctypes.c_void_p()
        call("rq_ctx_stream", h, ctypes.byref(s))
        self.stream = s
        n = ctypes.c_int()
        call("rq_ctx_num_cus", h, ctypes.byref(n))
        self.num_cus = n.value

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def sync(self) -> None:
        call("rq_sync", self._h, None)

    def close(self) -> None:
        if self._h:
            call("rq_ctx_destroy", self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


Context = WgpuContext


class UnifiedTensor:
    """A device buffer with a host-side shape (replaces ``UnifiedTensor``,
    lib.rs:79-241).  Memory is freed when the object is collected."""

    def __init__(self, ctx: WgpuContext, ptr: int, shape: Sequence[int], dtype: DType, owner: bool = True):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self._owner = owner

    # -- constructors (UnifiedTensor::new / ::empty, lib.rs:115-160) --------
    @classmethod
    def empty(cls, ctx: WgpuContext, shape: Sequence[int], dtype: DType = DType.FP32) -> "UnifiedTensor":
        nbytes = _prod(shape) * dtype.itemsize
        p = ctypes.c_void_p()
        call("rq_alloc", ctx.handle, nbytes, ctypes.byref(p))
        return cls(ctx, p.value or 0, shape, dtype)

    @classmethod
    def new(cls, ctx: WgpuContext, data, shape: Sequence[int] | None = None,
            dtype: DType | None = None) -> "UnifiedTensor":
        arr = np.asarray(data)
        if dtype is None:
            dtype = DType(arr.dtype.type) if arr.dtype.type in {d.value for d in DType} else DType.FP32
        arr = np.ascontiguousarray(arr, dtype=dtype.np)
        shape = tuple(arr.shape) if shape is None else tuple(shape)
        if _prod(shape) != arr.size:
            raise ValueError(f"shape {shape} does not match {arr.size} elements")
        t = cls.empty(ctx, shape, dtype)
        if arr.nbytes:
            call("rq_memcpy_h2d", ctx.handle, t.ptr, arr.ctypes.data, arr.nbytes, None)
        return t

    @property
    def numel(self) -> int:
        return _prod(self.shape)

    @property
    def nbytes(self) -> int:
        return self.numel * self.dtype.itemsize

    def reshaped(self, shape: Sequence[int]) -> "UnifiedTensor":
        """Aliases the buffer with a new shape (lib.rs:198-213)."""
        if _prod(shape) != self.numel:
            raise ValueError("reshape changes the element count")
        v = UnifiedTensor(self.ctx, self.ptr, shape, self.dtype, owner=False)
        v._base = self
        return v

    def to_vec(self, ctx: WgpuContext | None = None) -> np.ndarray:
        """Waits for queued work and reads the buffer back (lib.rs:215-240)."""
        ctx = ctx or self.ctx
        out = np.empty(self.shape, dtype=self.dtype.np)
        if out.nbytes:
            call("rq_memcpy_d2h", ctx.handle, out.ctypes.data, self.ptr, out.nbytes, None)
        return out

    def zero_(self) -> "UnifiedTensor":
        call("rq_memset", self.ctx.handle, self.ptr, 0, self.nbytes, None)
        return self

    def __del__(self):
        try:
            if self._owner and self.ptr and self.ctx.handle:
                call("rq_free", self.ctx.handle, self.ptr)
        except Exception:
            pass
        self.ptr = 0


@dataclass
class QuantizedTensor:
    """A quantized Linear weight W[n_out, k_in] on the device.

    The reference has no quantized tensor type: ``upload_quantized``
    (rusty-loader/src/lib.rs:155-218) keeps codes/scales/biases as raw
    buffers only long enough to dequantize them to f32.  Here they stay
    quantized and feed the fused kernels."""

    codes: UnifiedTensor
    scales: UnifiedTensor
    biases: UnifiedTensor | None
    n_out: int
    k_in: int
    format: int
    group: int
    prep: UnifiedTensor | None = None  # affine: the prefill GEMM's scale table (rq_qweight_prepare)

    @classmethod
    def rowwise(cls, ctx: WgpuContext, q: np.ndarray, scales: np.ndarray) -> "QuantizedTensor":
        """Signed int8 codes ``q[n_out, k_in]`` and one f32 scale per row."""
        q = np.ascontiguousarray(q, dtype=np.int8)
        n, k = q.shape
        s = np.ascontiguousarray(scales, dtype=np.float32).reshape(n)
        return cls(UnifiedTensor.new(ctx, q, dtype=DType.I8), UnifiedTensor.new(ctx, s, dtype=DType.FP32),
                   None, n, k, _lib.RQ_Q_ROWWISE_I8, 0)

    @classmethod
    def affine(cls, ctx: WgpuContext, u: np.ndarray, scales: np.ndarray, biases: np.ndarray | None,
               group: int = 64, prepare: bool = True) -> "QuantizedTensor":
        """The reference's affine format: unsigned codes ``u[n_out, k_in]``,
        f32 scale and bias per ``group`` consecutive flat elements.  With
        ``prepare`` the prefill GEMM's scale table is built once here (load
        time, as upload_quantized does its one-time work), so no GEMM call
        rebuilds it."""
        u = np.ascontiguousarray(u, dtype=np.uint8)
        n, k = u.shape
        s = UnifiedTensor.new(ctx, np.ascontiguousarray(scales, dtype=np.float32).ravel(), dtype=DType.FP32)
        b = None if biases is None else UnifiedTensor.new(
            ctx, np.ascontiguousarray(biases, dtype=np.float32).ravel(), dtype=DType.FP32)
        need = -(-n * k // group)
        if s.numel < need or (b is not None and b.numel < need):
            raise ValueError(f"{n}x{k} weight with group {group} needs {need} scales/biases")
        qt = cls(UnifiedTensor.new(ctx, u, dtype=DType.U8), s, b, n, k, _lib.RQ_Q_AFFINE_U8, group)
        if prepare:
            qt.prepare(ctx)
        return qt

    def prepare(self, ctx: WgpuContext, stream=None) -> None:
        """Builds the prefill GEMM's scale table of an affine weight
        (rq_qweight_prepare); nothing for weights that need none."""
        d = self.descriptor()
        d.prep = None
        nbytes = int(_lib.lib().rq_qweight_prep_bytes(ctypes.byref(d)))
        if nbytes == 0:
            self.prep = None
            return
        table = UnifiedTensor.empty(ctx, [nbytes // 4], DType.FP32)
        call("rq_qweight_prepare", ctx.handle, ctypes.byref(d), table.ptr, nbytes, _stream(stream))
        self.prep = table

    def dx_table(self, ctx: WgpuContext, stream=None) -> "UnifiedTensor | None":
        """The transposed-code table of the matrix-core input gradient
        (rq_qweight_dx_table), built on first use and kept with the weight;
        None when the weight is not served (see rq_qweight_dx_table_bytes)."""
        if getattr(self, "_dxt", None) is None:
            d = self.descriptor()
            nbytes = int(_lib.lib().rq_qweight_dx_table_bytes(ctypes.byref(d)))
            if nbytes == 0:
                return None
            table = UnifiedTensor.empty(ctx, [nbytes], DType.U8)
            call("rq_qweight_dx_table", ctx.handle, ctypes.byref(d), table.ptr, nbytes, _stream(stream))
            self._dxt = table
        return self._dxt

    def descriptor(self) -> rq_qweight:
        return rq_qweight(self.codes.ptr, self.scales.ptr, self.biases.ptr if self.biases is not None else None,
                          self.n_out, self.k_in, self.format, self.group,
                          self.prep.ptr if self.prep is not None else None)


_XDT = {DType.FP32: _lib.RQ_F32, DType.FP16: _lib.RQ_F16}


def _stream(stream):
    return None if stream is None else ctypes.c_void_p(stream if isinstance(stream, int) else stream.value)


class ComputeEngine:
    """Op surface of ``ComputeEngine`` (rusty-backend/src/lib.rs) for the
    quantized-linear path.  Every method enqueues work and returns."""

    def __init__(self, ctx: WgpuContext):
        self.ctx = ctx

    # ---- dequantization ---------------------------------------------------
    def dequantize(self, ctx: WgpuContext, input: UnifiedTensor, out: UnifiedTensor, stream=None) -> None:
        """lib.rs:4872-4899: ``out[4i+j] = byte j of input word i`` (unsigned,
        little-endian, no scale), for every input word that fits ``out``."""
        n_words = input.nbytes // 4
        call("rq_dequantize", ctx.handle, input.ptr, n_words, out.ptr, out.numel, _stream(stream))

    def affine_dequantize(self, ctx: WgpuContext, weight: UnifiedTensor, scales: UnifiedTensor,
                          biases: UnifiedTensor, out: UnifiedTensor, group: int = 64, fma: bool = False,
                          stream=None) -> None:
        """lib.rs:4939-4990: ``out[i] = f32(byte_i) * scales[i/64] + biases[i/64]``
        for every element of ``out`` (the reference's kernel hard-codes 64)."""
        n_groups = min(scales.numel, biases.numel if biases is not None else scales.numel)
        call("rq_affine_dequantize", ctx.handle, weight.ptr, weight.nbytes // 4, scales.ptr,
             biases.ptr if biases is not None else None, n_groups, out.ptr, out.numel, group,
             _lib.RQ_AFFINE_FMA if fma else 0, _stream(stream))

    def dequantize_weight(self, ctx: WgpuContext, w: QuantizedTensor, out: UnifiedTensor, stream=None) -> None:
        """Load-time dequantization of a QuantizedTensor to f32 [n_out, k_in]."""
        if out.numel != w.n_out * w.k_in:
            raise ValueError("output size does not match the weight")
        d = w.descriptor()
        call("rq_qweight_dequantize", ctx.handle, ctypes.byref(d), out.ptr, _stream(stream))

    # ---- f32 matmul family -----------------------------------------------
    def matmul(self, ctx: WgpuContext, a: UnifiedTensor, b: UnifiedTensor, out: UnifiedTensor,
               stream=None) -> None:
        """lib.rs:4403-4453: m, k, n = a.shape[0], a.shape[1], b.shape[1]."""
        m, k, n = a.shape[0], a.shape[1], b.shape[1]
        self._check_mm(a, b, out, (m, k), (k, n), (m, n))
        call("rq_matmul", ctx.handle, a.ptr, b.ptr, out.ptr, m, k, n, _stream(stream))

    def matmul_bt(self, ctx: WgpuContext, a: UnifiedTensor, b: UnifiedTensor, out: UnifiedTensor,
                  stream=None) -> None:
        """lib.rs:4299-4349: m, k, n = a.shape[0], a.shape[1], b.shape[0]."""
        m, k, n = a.shape[0], a.shape[1], b.shape[0]
        self._check_mm(a, b, out, (m, k), (n, k), (m, n))
        call("rq_matmul_bt", ctx.handle, a.ptr, b.ptr, out.ptr, m, k, n, _stream(stream))

    def matmul_at(self, ctx: WgpuContext, a: UnifiedTensor, b: UnifiedTensor, out: UnifiedTensor,
                  stream=None) -> None:
        """lib.rs:4351-4401: m, k, n = a.shape[1], a.shape[0], b.shape[1]."""
        m, k, n = a.shape[1], a.shape[0], b.shape[1]
        self._check_mm(a, b, out, (k, m), (k, n), (m, n))
        call("rq_matmul_at", ctx.handle, a.ptr, b.ptr, out.ptr, m, k, n, _stream(stream))

    @staticmethod
    def _check_mm(a, b, out, sa, sb, so):
        for t, s, nm in ((a, sa, "a"), (b, sb, "b"), (out, so, "out")):
            if t.dtype is not DType.FP32 or t.numel != _prod(s):
                raise ValueError(f"{nm}: expected f32 with {_prod(s)} elements for shape {s}, "
                                 f"got {t.dtype.name} {t.shape}")

    # ---- fused quantized linear -------------------------------------------
    def qmatmul(self, ctx: WgpuContext, x: UnifiedTensor, w: QuantizedTensor, out: UnifiedTensor,
                stream=None) -> None:
        """``out[m, n_out] = x[m, k_in] . deq(w)^T`` with dequantization fused
        into the product (what ``Linear::forward``, rusty-graph/src/lib.rs:69,
        computes on the reference's dequantized weight)."""
        if x.dtype not in _XDT or out.dtype not in _XDT:
            raise ValueError("x and out must be FP16 or FP32")
        m = x.numel // w.k_in if w.k_in else x.shape[0]
        if x.numel != m * w.k_in or out.numel != m * w.n_out:
            raise ValueError(f"x {x.shape} / out {out.shape} do not match weight [{w.n_out}, {w.k_in}]")
        d = w.descriptor()
        call("rq_qmatmul", ctx.handle, ctypes.byref(d), x.ptr, _XDT[x.dtype], out.ptr, _XDT[out.dtype], m,
             _stream(stream))

    def qmatmul_lora(self, ctx: WgpuContext, x: UnifiedTensor, w: QuantizedTensor, lora_a: UnifiedTensor,
                     lora_b: UnifiedTensor, out: UnifiedTensor, workspace: UnifiedTensor | None = None,
                     stream=None, tree: bool = False) -> None:
        """``Linear::forward`` with a LoRA adapter (rusty-graph/src/lib.rs:69-83):
        ``out = x . deq(w)^T + (x . A) . B``, A f32 [k_in, rank], B f32
        [rank, n_out], unscaled as the reference adds it.  ``tree``: x . A as
        a fixed-order reduction tree (rq_qmatmul_lora_ex, RQ_LORA_TREE) instead
        of the reference's k-ascending chain -- within f32 rounding of it, not
        its bits, and without the chain's k_in-step latency."""
        if x.dtype not in _XDT or out.dtype not in _XDT:
            raise ValueError("x and out must be FP16 or FP32")
        if lora_a.dtype is not DType.FP32 or lora_b.dtype is not DType.FP32:
            raise ValueError("the adapter's A and B must be FP32")
        m = x.numel // w.k_in if w.k_in else x.shape[0]
        rank = lora_a.numel // w.k_in if w.k_in else 0
        if x.numel != m * w.k_in or out.numel != m * w.n_out or lora_a.numel != w.k_in * rank \
                or lora_b.numel != rank * w.n_out:
            raise ValueError(f"x {x.shape} / A {lora_a.shape} / B {lora_b.shape} / out {out.shape} do not match "
                             f"weight [{w.n_out}, {w.k_in}]")
        flags = _lib.RQ_LORA_TREE if tree else 0
        need = _lib.lib().rq_qmatmul_lora_ex_workspace(m, w.k_in, w.n_out, rank, _XDT[x.dtype], _XDT[out.dtype],
                                                       flags)
        if workspace is None:
            workspace = UnifiedTensor.empty(ctx, [max(need, 1)], DType.U8)
        d = w.descriptor()
        if tree:
            call("rq_qmatmul_lora_ex", ctx.handle, ctypes.byref(d), x.ptr, _XDT[x.dtype], lora_a.ptr, lora_b.ptr,
                 rank, out.ptr, _XDT[out.dtype], m, flags, workspace.ptr, workspace.numel * workspace.dtype.itemsize,
                 _stream(stream))
        else:
            call("rq_qmatmul_lora", ctx.handle, ctypes.byref(d), x.ptr, _XDT[x.dtype], lora_a.ptr, lora_b.ptr, rank,
                 out.ptr, _XDT[out.dtype], m, workspace.ptr, workspace.numel * workspace.dtype.itemsize,
                 _stream(stream))

    def qmatmul_dx(self, ctx: WgpuContext, dy: UnifiedTensor, w: QuantizedTensor, dx: UnifiedTensor,
                   stream=None, mfma: bool = False, workspace: UnifiedTensor | None = None) -> None:
        """Input gradient of ``qmatmul`` with the weight frozen:
        ``dx[m, k_in] = dy[m, n_out] . deq(w)`` -- the ``grad_a`` of
        ``MatMulNode::backward`` (rusty-autograd/src/lib.rs:152-158).
        ``mfma``: on the matrix cores (rq_qmatmul_dx_mfma, per-row int8
        weights; the weight's transposed table is built on first use) -- the
        f32 bar, not the f32 chain's bit pattern."""
        if dy.dtype not in _XDT or dx.dtype not in _XDT:
            raise ValueError("dy and dx must be FP16 or FP32")
        m = dy.numel // w.n_out if w.n_out else dx.shape[0]
        if dy.numel != m * w.n_out or dx.numel != m * w.k_in:
            raise ValueError(f"dy {dy.shape} / dx {dx.shape} do not match weight [{w.n_out}, {w.k_in}]")
        d = w.descriptor()
        if not mfma:
            call("rq_qmatmul_dx", ctx.handle, ctypes.byref(d), dy.ptr, _XDT[dy.dtype], dx.ptr, _XDT[dx.dtype], m,
                 _stream(stream))
            return
        table = w.dx_table(ctx, stream)
        if table is None:
            raise ValueError(f"weight [{w.n_out}, {w.k_in}] is not served by the matrix-core input gradient")
        need = int(_lib.lib().rq_qmatmul_dx_mfma_workspace(m, w.n_out))
        if workspace is None:
            workspace = UnifiedTensor.empty(ctx, [max(need, 1)], DType.U8)
        call("rq_qmatmul_dx_mfma", ctx.handle, ctypes.byref(d), table.ptr, dy.ptr, _XDT[dy.dtype], dx.ptr,
             _XDT[dx.dtype], m, workspace.ptr, workspace.numel * workspace.dtype.itemsize, _stream(stream))

    def mlp_swiglu(self, ctx: WgpuContext, x: UnifiedTensor, gate: QuantizedTensor, up: QuantizedTensor,
                   down: QuantizedTensor, out: UnifiedTensor, h: UnifiedTensor | None = None,
                   stream=None) -> UnifiedTensor:
        """``MLP::forward`` (rusty-graph/src/lib.rs:317-323):
        ``out = down(silu(x . gate^T) * (x . up^T))``.  ``h`` is the fp16
        workspace (2 * m * I values); returned, its first m*I hold silu(g)*u."""
        m = x.numel // gate.k_in if gate.k_in else out.shape[0]
        if h is None:
            h = UnifiedTensor.empty(ctx, [2, m, gate.n_out], DType.FP16)
        if h.dtype is not DType.FP16 or h.numel < 2 * m * gate.n_out:
            raise ValueError("h must be an fp16 workspace of 2*m*I values")
        if out.numel != m * down.n_out:
            raise ValueError("out does not match [m, H]")
        dg, du, dd = gate.descriptor(), up.descriptor(), down.descriptor()
        call("rq_mlp_swiglu", ctx.handle, ctypes.byref(dg), ctypes.byref(du), ctypes.byref(dd), x.ptr,
             _XDT[x.dtype], h.ptr, out.ptr, _XDT[out.dtype], m, _stream(stream))
        return h
