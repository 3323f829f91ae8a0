"""Writes tests/golden/golden.npz: frozen input/output vectors of the hot path.

The reference's own tests hold no golden vectors for dequantize,
affine_dequantize or matmul (it is Rust + WGSL and cannot run here), so the
fixtures are:

* the two known answers the reference's examples state
  (rusty-loader/examples/load_and_run.rs:18-34: the f32 words of [1,2,3,4]
  dequantize to [0,0,128,63]; rusty-backend/examples/ops_test.rs:13-17: a
  2x2 times the identity gives [1,2,3,4]);
* small seeded cases computed by the CPU oracle (oracle/oracle.c, itself
  pinned by tests/test_oracle.py), frozen here so a later change to the
  oracle or to the device path is caught against fixed bytes: the
  dequantizers bit for bit (kernels.wgsl:153-166, 379-400, both roundings of
  u*s + b), the f32 matmul family in k-ascending fma order (kernels.wgsl:
  7-54, 234-252), and the f64 truth of the fused linear and the SwiGLU MLP
  (rusty-graph/src/lib.rs:69-83, 317-323) for the tolerance tests.

Usage: python tests/golden/make_golden.py   (rewrites golden.npz)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

OUT = HERE / "golden.npz"


def cases() -> dict[str, np.ndarray]:
    from oracle import oracle as orc
    from rusty_amd import synth

    d: dict[str, np.ndarray] = {}
    # a2 dequantize: known answer, then random words with a length guard (150 < 4 * 38)
    d["dq_ka_words"] = np.array([1.0, 2.0, 3.0, 4.0], np.float32).view(np.uint32)
    d["dq_ka_out"] = np.array([0.0, 0.0, 128.0, 63.0], np.float32)
    g = synth.rng(101)
    d["dq_words"] = g.integers(0, 2**32, 38, dtype=np.uint32)
    d["dq_out"] = orc.dequantize(d["dq_words"], 150)

    # a1 affine_dequantize: 3 x 100 codes (n % 64 != 0, n % 16 != 0), group 64, both roundings;
    # 5 x 30 with group 32 (n % 4 != 0 after flattening 150 -> byte tail)
    u, s, b = synth.affine_weight(synth.rng(102), 3, 100)
    d["af_u"], d["af_s"], d["af_b"] = u, s, b
    d["af_out"] = orc.affine_dequantize(u, s, b)
    d["af_out_fma"] = orc.affine_dequantize(u, s, b, fused=True)
    u32, s32, b32 = synth.affine_weight(synth.rng(103), 5, 30, group=32)
    d["af32_u"], d["af32_s"], d["af32_b"] = u32, s32, b32
    d["af32_out"] = orc.affine_dequantize(u32, s32, b32, group=32)

    # load-time dequantization of a per-row int8 weight
    q, sc = synth.rowwise_weight(synth.rng(104), 5, 48)
    d["rw_q"], d["rw_s"] = q, sc
    d["rw_out"] = orc.rowwise_dequantize(q, sc)

    # a3 / a4 / a4' f32 matmul family, k-ascending fma
    gm = synth.rng(105)
    d["mm_ka_a"] = np.array([[1, 2], [3, 4]], np.float32)
    d["mm_ka_out"] = np.array([[1, 2], [3, 4]], np.float32)
    d["mm_a"] = gm.standard_normal((5, 7), dtype=np.float32)
    d["mm_b"] = gm.standard_normal((7, 6), dtype=np.float32)
    d["mm_out"] = orc.matmul(d["mm_a"], d["mm_b"], fused=True)
    d["mmbt_b"] = gm.standard_normal((6, 7), dtype=np.float32)
    d["mmbt_out"] = orc.matmul_bt(d["mm_a"], d["mmbt_b"], fused=True)
    d["mmat_a"] = gm.standard_normal((7, 5), dtype=np.float32)
    d["mmat_out"] = orc.matmul_at(d["mmat_a"], d["mm_b"], fused=True)

    # fused linear: per-row int8 [48, 64] with fp16 X of 3 rows (decode) and
    # 40 rows (the prefill/generic path); affine u8 [48, 128], group 64
    gq = synth.rng(106)
    q, sc = synth.rowwise_weight(gq, 48, 64)
    d["ql_q"], d["ql_s"] = q, sc
    for m in (3, 40):
        x = synth.activations(gq, m, 64)
        d[f"ql_x{m}"] = x
        d[f"ql_y{m}"] = orc.qlinear_truth(q, sc, None, x.astype(np.float32), 0)
    u, s, b = synth.affine_weight(gq, 48, 128)
    xa = synth.activations(gq, 3, 128)
    d["qa_u"], d["qa_s"], d["qa_b"], d["qa_x"] = u, s, b, xa
    d["qa_y"] = orc.qlinear_truth(u, s, b, xa.astype(np.float32), 1, 64)

    # SwiGLU MLP, I = 96, H = 64, m = 2 (h rounded to fp16 as the device stores it)
    gs = synth.rng(107)
    wg, sg = synth.rowwise_weight(gs, 96, 64)
    wu, su = synth.rowwise_weight(gs, 96, 64)
    wd, sd = synth.rowwise_weight(gs, 64, 96)
    xs = synth.activations(gs, 2, 64)
    for k, v in dict(sw_wg=wg, sw_sg=sg, sw_wu=wu, sw_su=su, sw_wd=wd, sw_sd=sd, sw_x=xs).items():
        d[k] = v
    d["sw_y"] = orc.swiglu_truth(wg, sg, wu, su, wd, sd, xs.astype(np.float32), h_round_f16=True)
    return d


def main() -> None:
    np.savez_compressed(OUT, **cases())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
