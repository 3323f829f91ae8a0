"""MLX affine 8-bit safetensors -> device-resident quantized weights.

Host mirror of the reference's loader (rusty-loader/src/lib.rs): the
`QuantizationConfig` of a model's config.json (:27-32), `WeightsContext`
with `load_file` / `get_tensor_info` / `read_bytes` (:95-160) and
`upload_quantized` (:155-218).  What changes on the way to the device:

* `upload_quantized` returns a `QuantizedTensor` (codes, scales, biases stay
  quantized in HBM and feed the fused kernels) instead of dequantizing to an
  f32 tensor on every load; `upload_dequantized` keeps the reference's f32
  result for callers that want it.
* The logical shape is `[out, in]` (in = packed columns * 32 / bits); the
  reference allocates its output with the packed `[out, in/4]` shape (:172-174,
  206).
* Scales and biases may be F32, F16 or BF16 in the file (MLX stores them in the
  model dtype); they are widened to f32 on the host, exactly.  The reference
  reinterprets their bytes as f32 whatever their dtype (:186-187).
* `group_size`, `bits` and `mode` are honoured: 8-bit affine codes with any
  group size dividing `in` (a multiple of 16 for the fast kernels); the
  reference's kernel hard-codes group 64 (kernels.wgsl:395).

The safetensors container is parsed here directly (8-byte little-endian
header length, JSON header of name -> {dtype, shape, data_offsets}, raw
little-endian data), memory-mapped, so BF16 needs no numpy support and nothing
in the file is executed.
"""
from __future__ import annotations

import ctypes
import json
import mmap
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .engine import DType, QuantizedTensor, UnifiedTensor, WgpuContext
from . import _lib

_NP = {"F32": np.float32, "F16": np.float16, "U32": np.uint32, "U8": np.uint8, "I8": np.int8, "I32": np.int32,
       "F64": np.float64, "I64": np.int64, "U16": np.uint16, "I16": np.int16}
_SIZE = {"BF16": 2, **{k: np.dtype(v).itemsize for k, v in _NP.items()}}


class LoaderError(RuntimeError):
    """Missing weight, malformed file or unsupported quantization (the
    reference's LoaderError, rusty-loader/src/lib.rs:15-25)."""


@dataclass(frozen=True)
class QuantizationConfig:
    """`quantization` block of an MLX config.json (rusty-loader/src/lib.rs:27-32)."""
    group_size: int = 64
    bits: int = 8
    mode: str = "affine"

    @classmethod
    def from_json(cls, d: dict | None) -> "QuantizationConfig":
        d = d or {}
        return cls(int(d.get("group_size", 64)), int(d.get("bits", 8)), str(d.get("mode", "affine")))


def load_config(path) -> dict:
    """A model's config.json as a dict, with `quantization` parsed
    (ModelLoader::load_config, rusty-loader/src/lib.rs:75-80)."""
    with open(path) as f:
        cfg = json.load(f)
    if "quantization" in cfg:
        cfg["quantization"] = QuantizationConfig.from_json(cfg["quantization"])
    return cfg


def _widen(raw: np.ndarray, dtype: str) -> np.ndarray:
    """F32 / F16 / BF16 -> f32, exactly."""
    if dtype == "BF16":
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype in ("F32", "F16"):
        return raw.astype(np.float32)
    raise LoaderError(f"scales/biases must be F32, F16 or BF16, not {dtype}")


class _File:
    def __init__(self, path: Path):
        self.path = path
        self._fh = open(path, "rb")
        try:
            self.map = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:  # empty file
            raise LoaderError(f"{path}: not a safetensors file ({e})") from e
        if len(self.map) < 8:
            raise LoaderError(f"{path}: not a safetensors file")
        (n,) = struct.unpack("<Q", self.map[:8])
        if n > len(self.map) - 8:
            raise LoaderError(f"{path}: header length {n} past the end of the file")
        try:
            header = json.loads(self.map[8:8 + n].decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise LoaderError(f"{path}: bad header ({e})") from e
        self.base = 8 + n
        self.tensors = {k: v for k, v in header.items() if k != "__metadata__"}
        for name, t in self.tensors.items():
            b, e = t["data_offsets"]
            count = int(np.prod(t["shape"], dtype=np.int64)) if t["shape"] else 1
            if t["dtype"] not in _SIZE:
                continue  # dtypes this path never reads are left alone
            if not (0 <= b <= e <= len(self.map) - self.base) or e - b != count * _SIZE[t["dtype"]]:
                raise LoaderError(f"{path}: tensor {name} has inconsistent offsets")

    def array(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        b, e = t["data_offsets"]
        dt = np.uint16 if t["dtype"] == "BF16" else _NP.get(t["dtype"])
        if dt is None:
            raise LoaderError(f"tensor {name}: dtype {t['dtype']} is not supported")
        return np.frombuffer(self.map, dtype=dt, count=(e - b) // np.dtype(dt).itemsize,
                             offset=self.base + b).reshape(t["shape"])

    def close(self):
        try:
            self.map.close()
        except BufferError:
            pass  # arrays from read_bytes still view it; it unmaps when the last one goes
        self._fh.close()


class WeightsContext:
    """Memory-mapped safetensors files and a weight-name index
    (rusty-loader/src/lib.rs:95-125)."""

    def __init__(self):
        self._files: dict[str, _File] = {}
        self.weight_map: dict[str, str] = {}

    def load_file(self, path) -> None:
        f = _File(Path(path))
        self._files[f.path.name] = f
        for name in f.tensors:
            self.weight_map[name] = f.path.name

    def _lookup(self, name: str) -> tuple[_File, dict]:
        fname = self.weight_map.get(name)
        if fname is None:
            raise LoaderError(f"Weight not found: {name}")
        f = self._files[fname]
        return f, f.tensors[name]

    def get_tensor_info(self, name: str):
        """(shape, dtype string) or None (rusty-loader/src/lib.rs:127-137)."""
        if name not in self.weight_map:
            return None
        _, t = self._lookup(name)
        return list(t["shape"]), t["dtype"]

    def read_bytes(self, name: str):
        """(raw little-endian data as a read-only array view, shape)
        (rusty-loader/src/lib.rs:142-157)."""
        f, t = self._lookup(name)
        return f.array(name), list(t["shape"])

    def _quantized_host(self, name: str, q: QuantizationConfig):
        if q.mode != "affine" or q.bits != 8:
            raise LoaderError(f"{name}: only 8-bit affine quantization is supported (got {q.bits}-bit {q.mode})")
        w, wshape = self.read_bytes(f"{name}.weight")
        wdt = self._lookup(f"{name}.weight")[1]["dtype"]
        if len(wshape) != 2 or wdt not in ("U32", "U8"):
            raise LoaderError(f"{name}.weight: expected packed U32 [out, in/4] or U8 [out, in], got {wdt} {wshape}")
        n_out = wshape[0]
        codes = np.array(w, copy=True).view(np.uint8).reshape(n_out, -1)  # little-endian: element order
        k_in = codes.shape[1]
        if q.group_size <= 0 or k_in % q.group_size != 0:
            raise LoaderError(f"{name}: in = {k_in} is not a multiple of group_size {q.group_size}")
        n_groups = n_out * k_in // q.group_size
        out = []
        for part in ("scales", "biases"):
            a, shape = self.read_bytes(f"{name}.{part}")
            dt = self._lookup(f"{name}.{part}")[1]["dtype"]
            if int(np.prod(shape)) != n_groups:
                raise LoaderError(f"{name}.{part}: {int(np.prod(shape))} values, expected {n_groups} "
                                  f"([{n_out}, {k_in // q.group_size}])")
            out.append(_widen(np.ascontiguousarray(a), dt).reshape(-1))
        return codes, out[0], out[1]

    def upload_quantized(self, name: str, ctx: WgpuContext, quant: QuantizationConfig | None = None
                         ) -> QuantizedTensor:
        """`{name}.weight/.scales/.biases` -> a device `QuantizedTensor`
        [out, in] in the reference's affine format, ready for the fused
        kernels (rusty-loader/src/lib.rs:155-218 without the f32 step)."""
        codes, s, b = self._quantized_host(name, quant or QuantizationConfig())
        g = (quant or QuantizationConfig()).group_size
        return QuantizedTensor.affine(ctx, codes, s, b, group=g)

    def upload_dequantized(self, name: str, ctx: WgpuContext, quant: QuantizationConfig | None = None
                           ) -> UnifiedTensor:
        """The reference's result: an f32 [out, in] tensor dequantized on the
        device (affine_dequantize, kernels.wgsl:379-400)."""
        qt = self.upload_quantized(name, ctx, quant)
        out = UnifiedTensor.empty(ctx, [qt.n_out, qt.k_in], DType.FP32)
        _lib.call("rq_qweight_dequantize", ctx.handle, ctypes.byref(qt.descriptor()), out.ptr, None)
        return out

    def close(self) -> None:
        for f in self._files.values():
            f.close()
        self._files.clear()
        self.weight_map.clear()


def save_safetensors(path, tensors: dict[str, tuple[str, np.ndarray]]) -> None:
    """Writes name -> (dtype string, array) as a safetensors file (BF16 given
    as uint16 bit patterns).  Used to produce MLX-layout test files."""
    header, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)
