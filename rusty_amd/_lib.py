"""ctypes binding of the C ABI declared in ``include/rusty_hip.h``.

The shared library ``rusty_amd/librusty_hip.so`` is built in-tree by
``rusty_amd/build.py`` (or ``__graft_entry__.build()``).  There is no
fallback: if the library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import re
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "librusty_hip.so"
HEADER = PKG.parent / "include" / "rusty_hip.h"

RQ_OK = 0
RQ_ERR_INVALID_ARGUMENT = -1
RQ_ERR_SHAPE = -2
RQ_ERR_UNSUPPORTED = -3
RQ_ERR_HIP = -4
RQ_ERR_NO_DEVICE = -5
RQ_ERR_ALLOC = -6

RQ_F32 = 0
RQ_F16 = 1
RQ_Q_ROWWISE_I8 = 0
RQ_Q_AFFINE_U8 = 1
RQ_AFFINE_FMA = 1
RQ_LORA_TREE = 1


class rq_qweight(ctypes.Structure):
    _fields_ = [
        ("codes", c_void_p),
        ("scales", c_void_p),
        ("biases", c_void_p),
        ("n_out", c_int64),
        ("k_in", c_int64),
        ("format", c_int32),
        ("group", c_int32),
        ("prep", c_void_p),
    ]


class rq_llama_config(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32),
        ("hidden", c_int32),
        ("n_heads", c_int32),
        ("n_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("intermediate", c_int32),
        ("vocab", c_int32),
        ("max_seq", c_int32),
        ("norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
    ]


class rq_llama_layer(ctypes.Structure):
    _fields_ = [
        ("attn_norm", c_void_p),
        ("q", rq_qweight),
        ("k", rq_qweight),
        ("v", rq_qweight),
        ("o", rq_qweight),
        ("mlp_norm", c_void_p),
        ("gate", rq_qweight),
        ("up", rq_qweight),
        ("down", rq_qweight),
    ]


class rq_llama_weights(ctypes.Structure):
    _fields_ = [
        ("embed", c_void_p),
        ("layers", POINTER(rq_llama_layer)),
        ("final_norm", c_void_p),
        ("lm_head", rq_qweight),
    ]


_P = c_void_p
# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
_SIGNATURES = {
    "rq_ctx_create": [c_int, POINTER(c_void_p)],
    "rq_ctx_destroy": [_P],
    "rq_ctx_stream": [_P, POINTER(c_void_p)],
    "rq_ctx_num_cus": [_P, POINTER(c_int)],
    "rq_sync": [_P, _P],
    "rq_device_delay": [_P, c_uint32, _P],
    "rq_stream_probe": [_P, _P, c_size_t, c_size_t, c_int, _P, c_int, _P],
    "rq_fma_chain_probe": [_P, ctypes.c_int64, _P, _P],
    "rq_device_clock": [_P, _P, POINTER(ctypes.c_uint64), _P],
    "rq_status_string": [c_int],
    "rq_last_error": [],
    "rq_alloc": [_P, c_size_t, POINTER(c_void_p)],
    "rq_free": [_P, _P],
    "rq_memcpy_h2d": [_P, _P, _P, c_size_t, _P],
    "rq_memcpy_d2h": [_P, _P, _P, c_size_t, _P],
    "rq_memcpy_d2d": [_P, _P, _P, c_size_t, _P],
    "rq_memset": [_P, _P, c_int, c_size_t, _P],
    "rq_dequantize": [_P, _P, c_size_t, _P, c_size_t, _P],
    "rq_affine_dequantize": [_P, _P, c_size_t, _P, _P, c_size_t, _P, c_size_t, c_uint32, c_uint32, _P],
    "rq_qweight_dequantize": [_P, POINTER(rq_qweight), _P, _P],
    "rq_qweight_prep_bytes": [POINTER(rq_qweight)],
    "rq_qweight_prepare": [_P, POINTER(rq_qweight), _P, c_size_t, _P],
    "rq_matmul": [_P, _P, _P, _P, c_int64, c_int64, c_int64, _P],
    "rq_matmul_bt": [_P, _P, _P, _P, c_int64, c_int64, c_int64, _P],
    "rq_matmul_at": [_P, _P, _P, _P, c_int64, c_int64, c_int64, _P],
    "rq_qmatmul": [_P, POINTER(rq_qweight), _P, c_int, _P, c_int, c_int64, _P],
    "rq_mlp_swiglu": [_P, POINTER(rq_qweight), POINTER(rq_qweight), POINTER(rq_qweight), _P, c_int, _P, _P, c_int,
                      c_int64, _P],
    "rq_mlp_swiglu_noalloc": [_P, POINTER(rq_qweight), POINTER(rq_qweight), POINTER(rq_qweight), _P, c_int, _P,
                              c_int, c_int64, _P],
    "rq_qmatmul_dx": [_P, POINTER(rq_qweight), _P, c_int, _P, c_int, c_int64, _P],
    "rq_qweight_dx_table_bytes": [POINTER(rq_qweight)],
    "rq_qweight_dx_table": [_P, POINTER(rq_qweight), _P, c_size_t, _P],
    "rq_qmatmul_dx_mfma_workspace": [c_int64, c_int64],
    "rq_qmatmul_dx_mfma": [_P, POINTER(rq_qweight), _P, _P, c_int, _P, c_int, c_int64, _P, c_size_t, _P],
    "rq_llama_create": [_P, POINTER(rq_llama_config), POINTER(rq_llama_weights), POINTER(c_void_p)],
    "rq_llama_destroy": [_P],
    "rq_llama_prefill": [_P, POINTER(c_int32), c_int32, _P],
    "rq_llama_decode": [_P, c_int32, _P],
    "rq_qmatmul_lora_workspace": [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int],
    "rq_qmatmul_lora": [_P, POINTER(rq_qweight), _P, c_int, _P, _P, ctypes.c_int64, _P, c_int, ctypes.c_int64, _P,
                        c_size_t, _P],
    "rq_qmatmul_lora_ex_workspace": [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int,
                                     c_uint32],
    "rq_qmatmul_lora_ex": [_P, POINTER(rq_qweight), _P, c_int, _P, _P, ctypes.c_int64, _P, c_int, ctypes.c_int64,
                           c_uint32, _P, c_size_t, _P],
    "rq_llama_set_graph": [_P, c_int],
    "rq_llama_set_prefill": [_P, c_int32],
    "rq_llama_tokens": [_P, POINTER(c_int32), c_int32, POINTER(c_int32), _P],
    "rq_llama_logits": [_P, POINTER(ctypes.c_float), _P],
}
_RESTYPES = {"rq_status_string": c_char_p, "rq_last_error": c_char_p, "rq_qmatmul_lora_workspace": c_size_t,
             "rq_qmatmul_lora_ex_workspace": c_size_t, "rq_qweight_prep_bytes": c_size_t,
             "rq_qweight_dx_table_bytes": c_size_t, "rq_qmatmul_dx_mfma_workspace": c_size_t}


class RqError(RuntimeError):
    """A non-zero rq_status returned by the library."""

    def __init__(self, status: int, where: str, message: str):
        self.status = status
        name = _lib.rq_status_string(status).decode() if _lib is not None else str(status)
        super().__init__(f"{where}: {name} ({status}): {message}")


_lib: ctypes.CDLL | None = None


def header_symbols() -> list[str]:
    """Names of every function declared in include/rusty_hip.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rq_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """Loads librusty_hip.so (once) and declares every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the HIP library is required: there is no CPU fallback)")
    handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, c_int)
    _lib = handle
    return handle


def check(status: int, where: str) -> None:
    if status != RQ_OK:
        msg = _lib.rq_last_error().decode(errors="replace") if _lib is not None else ""
        raise RqError(status, where, msg)


def call(name: str, *args) -> None:
    """Calls an entry point and raises RqError on a non-zero status."""
    check(getattr(lib(), name)(*args), name)
