"""Seeded synthetic inputs of the benchmark configurations.

Host arrays only (numpy ``default_rng`` / PCG64); the same seed gives the same
bytes on every machine, so the device path and the CPU oracle see identical
inputs.

* per-row int8 weight: codes uniform in [-127, 127], f32 scale per output row
  ~ U(0.001, 0.02)
* affine u8 weight (the reference's format): codes uniform in [0, 255], f32
  scale per group ~ U(0.001, 0.02), bias = -128*scale + U(-0.01, 0.01)
* activations ~ N(0, sigma), rounded to fp16 (round-to-nearest-even) or kept f32.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def rowwise_weight(g: np.random.Generator, n_out: int, k_in: int):
    q = g.integers(-127, 128, size=(n_out, k_in), dtype=np.int8)
    s = g.uniform(0.001, 0.02, size=n_out).astype(np.float32)
    return q, s


def affine_weight(g: np.random.Generator, n_out: int, k_in: int, group: int = 64):
    u = g.integers(0, 256, size=(n_out, k_in), dtype=np.uint8)
    n_groups = -(-n_out * k_in // group)
    s = g.uniform(0.001, 0.02, size=n_groups).astype(np.float32)
    b = (-128.0 * s.astype(np.float64) + g.uniform(-0.01, 0.01, size=n_groups)).astype(np.float32)
    return u, s, b


def activations(g: np.random.Generator, m: int, k: int, sigma: float = 1.0, dtype=np.float16) -> np.ndarray:
    x = g.standard_normal((m, k), dtype=np.float32) * np.float32(sigma)
    return x.astype(dtype)
