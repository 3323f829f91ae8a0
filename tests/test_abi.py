"""CPU checks of the C ABI: the library loads, exports every symbol that
include/rusty_hip.h declares, and its non-compute entry points behave
(status strings, argument errors, no-device error).  No kernel runs here."""
import ctypes
import subprocess

import pytest

from rusty_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _lib.header_symbols()
    assert len(declared) >= 20
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in rusty_hip.h but not exported: {missing}"
    # and the binding declares a signature for each of them
    assert set(declared) == set(_lib._SIGNATURES), set(declared) ^ set(_lib._SIGNATURES)


def test_exports_match_nm():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T rq_" in ln}
    assert exported == set(_lib.header_symbols())


def test_status_strings():
    lib = _lib.lib()
    assert lib.rq_status_string(0) == b"RQ_OK"
    assert lib.rq_status_string(-2) == b"RQ_ERR_SHAPE"
    assert lib.rq_status_string(12345) == b"RQ_ERR_UNKNOWN"


def test_null_arguments_rejected_without_device():
    lib = _lib.lib()
    assert lib.rq_ctx_create(0, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_sync(None, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert b"null context" in lib.rq_last_error()
    assert lib.rq_qmatmul(None, None, None, 0, None, 0, 1, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_ctx_destroy(None) == _lib.RQ_OK


def test_struct_layout_matches_header():
    # rq_qweight: 3 pointers, 2 int64, 2 int32 -> 48 bytes, no padding surprises
    assert ctypes.sizeof(_lib.rq_qweight) == 48
    assert _lib.rq_qweight.n_out.offset == 24 and _lib.rq_qweight.format.offset == 40
