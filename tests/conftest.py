import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


@pytest.fixture(scope="session")
def ctx():
    """One device context for the whole GPU session (fails loudly without a gfx950)."""
    from rusty_amd import WgpuContext

    c = WgpuContext(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def engine(ctx):
    from rusty_amd import ComputeEngine

    return ComputeEngine(ctx)


def f16_tol_check(y_dev: np.ndarray, truth: np.ndarray, rel: float = 2e-3, absn: float = 2e-3):
    """fp16-output bar: |dy| <= rel*|y| + absn*max|y| elementwise, vs f64 truth.
    Returns (max_abs, max_rel, ok)."""
    y = y_dev.astype(np.float64)
    d = np.abs(y - truth)
    scale = np.abs(truth).max() if truth.size else 0.0
    bound = rel * np.abs(truth) + absn * scale
    max_rel = float((d / np.maximum(np.abs(truth), 1e-30)).max()) if truth.size else 0.0
    return float(d.max()) if d.size else 0.0, max_rel, bool(np.all(d <= bound))


def f32_norm_check(y_dev: np.ndarray, truth: np.ndarray, tol: float = 1e-5):
    """f32-output bar: max|dy| / max|y| <= tol, vs f64 truth."""
    d = np.abs(y_dev.astype(np.float64) - truth)
    scale = np.abs(truth).max() if truth.size else 1.0
    r = float(d.max() / scale) if d.size and scale > 0 else 0.0
    return float(d.max()) if d.size else 0.0, r, r <= tol
