import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture
def rng():
    return np.random.default_rng(12345)


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the library initialised; skips when no GPU is visible."""
    if not gpu_available():
        pytest.skip("no GPU visible")
    import torch
    import fufft_amd as ff
    ff.init(0)
    return torch.device("cuda:0")


def crandn(rng, shape, scale=1.0):
    return ((rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) * scale).astype(np.complex64)


def cuniform(rng, shape, lo=-1.0, hi=1.0):
    return (rng.uniform(lo, hi, shape) + 1j * rng.uniform(lo, hi, shape)).astype(np.complex64)


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def lane_major(fdr, n, v):
    """Digit-order filters or spectra (rows of n) in the lane-major pair layout
    (FUFFT_LAYOUT_LANE): lane L's slots L*v + 2m and L*v + 2m + 1 at positions
    2(L + m*T) and 2(L + m*T) + 1, T = n // v."""
    t = n // v
    f = np.asarray(fdr).reshape(-1, t, v // 2, 2)
    return np.ascontiguousarray(f.transpose(0, 2, 1, 3)).reshape(np.shape(fdr))


def bperm(fdr, n, v):
    """Digit-order filters (rows of n) in the reference's bperm layout
    (FUFFT_LAYOUT_BPERM, verify_kernel.cpp:1381-1387): slot L*v + k at L + k*T."""
    t = n // v
    return np.ascontiguousarray(np.asarray(fdr).reshape(-1, t, v).transpose(0, 2, 1)).reshape(np.shape(fdr))


def lane_slot(c, n, v):
    """The digit-order slot that lane-major position c holds (inverse of lane_major)."""
    t = n // v
    return ((c // 2) % t) * v + 2 * ((c // 2) // t) + c % 2


def cols_to_dr(x, h, w):
    """A 2D filter or spectrum in the library's column order (lane-major rows,
    fufft_plan2d_column_order) re-ordered to the reference's digit order,
    slot (r, c) = bin (mixedrev_h(r), mixedrev_w(c)), which the oracle uses."""
    import fufft_amd as ff
    slot = ff.column_order2d(h, w)
    a = np.asarray(x).reshape(-1, h, w)
    out = np.empty_like(a)
    out[:, :, slot] = a
    return out.reshape(np.shape(x))


def filt2d_dr(x, h, w, layout):
    """A 2D filter or spectrum planned in `layout` ("dr": the reference's
    order already; "lane": the library's column order) in the reference's
    order, slot (r, c) = bin (mixedrev_h(r), mixedrev_w(c)), which the oracle
    reads."""
    return np.asarray(x) if layout == "dr" else cols_to_dr(x, h, w)
