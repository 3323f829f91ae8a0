"""MLX affine safetensors loading (rusty_amd/loader.py) -- host side, no GPU.

The files are written here in the MLX layout the reference's loader reads
(rusty-loader/src/lib.rs:155-218): `{name}.weight` U32 [out, in/4] holding four
little-endian 8-bit codes per word, `{name}.scales` / `{name}.biases`
[out, in/group] in the model dtype.
"""
import json

import numpy as np
import pytest

from rusty_amd.loader import LoaderError, QuantizationConfig, WeightsContext, load_config, save_safetensors


def mlx_file(path, name, codes, scales, biases, sdt="F16"):
    enc = {"F16": lambda a: a.astype(np.float16), "F32": lambda a: a.astype(np.float32),
           "BF16": lambda a: (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)}[sdt]
    save_safetensors(path, {f"{name}.weight": ("U32", codes.view(np.uint32)),
                            f"{name}.scales": (sdt, enc(scales)), f"{name}.biases": (sdt, enc(biases)),
                            "other.norm": ("F16", np.ones(4, np.float16))})


def test_packing_order_and_shapes(tmp_path):
    # word 0x04030201 holds codes 1, 2, 3, 4: byte j of a word is (w >> 8j) & 0xFF,
    # the reference kernel's unpacking (kernels.wgsl:393-397)
    words = np.array([[0x04030201, 0xFFFEFDFC]], dtype=np.uint32)
    save_safetensors(tmp_path / "m.safetensors", {
        "l.weight": ("U32", words), "l.scales": ("F32", np.array([[1.0]], np.float32)),
        "l.biases": ("F32", np.array([[0.0]], np.float32))})
    wc = WeightsContext()
    wc.load_file(tmp_path / "m.safetensors")
    assert wc.get_tensor_info("l.weight") == ([1, 2], "U32")
    assert wc.get_tensor_info("missing") is None
    codes, s, b = wc._quantized_host("l", QuantizationConfig(group_size=8))
    assert codes.tolist() == [[1, 2, 3, 4, 0xFC, 0xFD, 0xFE, 0xFF]] and codes.shape == (1, 8)


@pytest.mark.parametrize("sdt", ["F16", "BF16", "F32"])
def test_scales_widened_exactly(tmp_path, sdt):
    g = np.random.default_rng(3)
    codes = g.integers(0, 256, (6, 128), dtype=np.uint8)
    s = g.uniform(0.001, 0.02, (6, 2))
    b = -128 * s + g.uniform(-0.01, 0.01, (6, 2))
    mlx_file(tmp_path / "a.safetensors", "model.layers.0.mlp.up_proj", codes, s, b, sdt)
    wc = WeightsContext()
    wc.load_file(tmp_path / "a.safetensors")
    got_c, got_s, got_b = wc._quantized_host("model.layers.0.mlp.up_proj", QuantizationConfig(64, 8, "affine"))
    assert np.array_equal(got_c, codes)
    if sdt == "F16":
        want_s, want_b = s.astype(np.float16).astype(np.float32), b.astype(np.float16).astype(np.float32)
    elif sdt == "F32":
        want_s, want_b = s.astype(np.float32), b.astype(np.float32)
    else:  # bf16 = the top 16 bits of the f32 pattern (truncated on write above), widened back exactly
        want_s = ((s.astype(np.float32).view(np.uint32) >> 16) << 16).view(np.float32)
        want_b = ((b.astype(np.float32).view(np.uint32) >> 16) << 16).view(np.float32)
    assert np.array_equal(got_s, want_s.ravel()) and np.array_equal(got_b, want_b.ravel())
    wc.close()


def test_errors(tmp_path):
    g = np.random.default_rng(4)
    codes = g.integers(0, 256, (4, 64), dtype=np.uint8)
    mlx_file(tmp_path / "e.safetensors", "w", codes, np.ones((4, 1)), np.zeros((4, 1)))
    wc = WeightsContext()
    wc.load_file(tmp_path / "e.safetensors")
    with pytest.raises(LoaderError, match="Weight not found: nope.weight"):
        wc._quantized_host("nope", QuantizationConfig())
    with pytest.raises(LoaderError, match="only 8-bit affine"):
        wc._quantized_host("w", QuantizationConfig(64, 4, "affine"))
    with pytest.raises(LoaderError, match="not a multiple of group_size"):
        wc._quantized_host("w", QuantizationConfig(48, 8, "affine"))
    with pytest.raises(LoaderError, match="expected 8"):
        wc._quantized_host("w", QuantizationConfig(32, 8, "affine"))  # file holds 4 scales, 8 needed
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\xff" * 16)
    with pytest.raises(LoaderError):
        WeightsContext().load_file(bad)
    trunc = tmp_path / "trunc.safetensors"
    trunc.write_bytes((tmp_path / "e.safetensors").read_bytes()[:-10])
    with pytest.raises(LoaderError, match="inconsistent offsets"):
        WeightsContext().load_file(trunc)


def test_load_config(tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps({"hidden_size": 2048, "quantization": {"group_size": 32, "bits": 8, "mode": "affine"}}))
    cfg = load_config(p)
    assert cfg["hidden_size"] == 2048 and cfg["quantization"] == QuantizationConfig(32, 8, "affine")
