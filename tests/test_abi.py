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
    assert lib.rq_device_delay(None, 10, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert b"null context" in lib.rq_last_error()
    assert lib.rq_qmatmul(None, None, None, 0, None, 0, 1, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert lib.rq_ctx_destroy(None) == _lib.RQ_OK


def test_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors have the sizes and field offsets a C compiler gives
    the header's structs (compiled and printed by gcc)."""
    import shutil
    import subprocess
    from pathlib import Path

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    root = Path(__file__).resolve().parent.parent
    src = tmp_path / "layout.c"
    src.write_text("""#include <stdio.h>
#include <stddef.h>
#include "rusty_hip.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu\\n", sizeof(rq_qweight), offsetof(rq_qweight, n_out),
           offsetof(rq_qweight, format), offsetof(rq_qweight, group), offsetof(rq_qweight, prep),
           sizeof(rq_llama_layer));
    printf("%zu %zu %zu\\n", sizeof(rq_llama_config), sizeof(rq_llama_weights), offsetof(rq_llama_weights, lm_head));
    return 0;
}
""")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", "-I", str(root / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    q = _lib.rq_qweight
    assert [int(v) for v in out] == [ctypes.sizeof(q), q.n_out.offset, q.format.offset, q.group.offset,
                                     q.prep.offset, ctypes.sizeof(_lib.rq_llama_layer),
                                     ctypes.sizeof(_lib.rq_llama_config), ctypes.sizeof(_lib.rq_llama_weights),
                                     _lib.rq_llama_weights.lm_head.offset]
    assert ctypes.sizeof(q) == 56  # 3 pointers, 2 int64, 2 int32, the table pointer


def _build_c_example(tmp_path):
    import shutil
    import subprocess
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "abi_example"
    subprocess.run([gcc, "-std=c99", "-O2", "-Wall", "-Werror", "-I", str(root / "include"),
                    str(root / "tests" / "c" / "abi_example.c"), "-L", str(root / "rusty_amd"), "-lrusty_hip",
                    "-Wl,-rpath," + str(root / "rusty_amd"), "-lm", "-o", str(exe)], check=True)
    return exe


def test_c_client_builds_against_header(tmp_path):
    """The header is plain C (c99, no HIP or C++ includes) and links to the library."""
    assert _build_c_example(tmp_path).exists()


@pytest.mark.gpu
def test_c_client_runs(tmp_path):
    import subprocess

    r = subprocess.run([str(_build_c_example(tmp_path))], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "abi_example: OK" in r.stdout


def test_integration_binding_lists_every_entry_point():
    """The integration guide's Rust `extern "C"` block (the binding a maintainer
    adds on the reference side) declares exactly the header's functions."""
    import re
    from pathlib import Path

    text = (Path(__file__).resolve().parent.parent / "INTEGRATION.md").read_text()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    bound = set(re.findall(r"pub fn (rq_[a-z0-9_]+)\s*\(", block))
    assert bound == set(_lib.header_symbols()), bound ^ set(_lib.header_symbols())


def test_workspace_and_table_sizes_without_device():
    """The size queries of the tree LoRA and the matrix-core input gradient are
    host arithmetic: the documented formulas, 0 for what is not served."""
    lib = _lib.lib()
    F16, F32, TREE = _lib.RQ_F16, _lib.RQ_F32, _lib.RQ_LORA_TREE
    m, k, n, rank = 3, 1000, 512, 16
    chain = lib.rq_qmatmul_lora_workspace(m, k, n, rank, F16, F16)
    assert lib.rq_qmatmul_lora_ex_workspace(m, k, n, rank, F16, F16, 0) == chain
    assert chain == (m * k + m * rank + m * n) * 4 + 3 * 256  # x f32 copy, t, the f32 product
    # tree: m * rank partials for each of ceil(k / 256) slices, then the f32 product
    assert lib.rq_qmatmul_lora_ex_workspace(m, k, n, rank, F16, F16, TREE) == (m * rank * 4 + m * n) * 4 + 3 * 256
    assert lib.rq_qmatmul_lora_ex_workspace(m, k, n, rank, F32, F32, TREE) == m * rank * 4 * 4 + 3 * 256
    # past rank 64 the tree flag keeps the chain's workspace
    assert lib.rq_qmatmul_lora_ex_workspace(m, k, n, 70, F16, F16, TREE) == \
        lib.rq_qmatmul_lora_workspace(m, k, n, 70, F16, F16)
    assert lib.rq_qmatmul_lora_ex_workspace(-1, k, n, rank, F16, F16, TREE) == 0
    # the input gradient: fp16 halves of dY (2 m n values) then m row factors
    assert lib.rq_qmatmul_dx_mfma_workspace(5, 96) == ((5 * 96 * 4 + 255) // 256) * 256 + 5 * 4
    assert lib.rq_qmatmul_dx_mfma_workspace(-1, 96) == 0

    def desc(fmt, n_out, k_in, codes=4096):
        return _lib.rq_qweight(codes, 4096, None, n_out, k_in, fmt, 64 if fmt else 0, None)

    w = desc(_lib.RQ_Q_ROWWISE_I8, 96, 48)
    assert lib.rq_qweight_dx_table_bytes(ctypes.byref(w)) == ((2 * 96 * 48 + 255) // 256) * 256 + 48 * 4
    for bad in (desc(_lib.RQ_Q_AFFINE_U8, 96, 64), desc(_lib.RQ_Q_ROWWISE_I8, 48, 64),
                desc(_lib.RQ_Q_ROWWISE_I8, 96, 40), desc(_lib.RQ_Q_ROWWISE_I8, 96, 48, codes=4100)):
        assert lib.rq_qweight_dx_table_bytes(ctypes.byref(bad)) == 0
    assert lib.rq_qweight_dx_table_bytes(None) == 0
