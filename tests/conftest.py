"""Shared pytest configuration.

Markers: `gpu` - needs a ROCm device (run with `-m gpu` on an MI355X);
everything else runs on the CPU. A GPU test on a machine without a device is
skipped; on a machine with one, a missing kernel library is an error.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def _gpu_present() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def hip():
    """The kernel library, loaded (raises if it is not built)."""
    from ttspipe_amd import _lib

    return _lib.load()


@pytest.fixture(scope="session")
def selftest():
    """The numerics self-test library (tests/csrc/selftest.hip), loaded."""
    import ctypes

    from tests import build_selftest

    if not build_selftest.LIB.exists():
        raise RuntimeError(f"{build_selftest.LIB} is not built; run `python -m tests.build_selftest`")
    lib = ctypes.CDLL(str(build_selftest.LIB))
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.ttsp_selftest_math.argtypes = [vp, i, i, vp, vp]
    lib.ttsp_selftest_fma16.argtypes = [vp, vp, vp, i, vp, vp]
    lib.ttsp_selftest_math.restype = lib.ttsp_selftest_fma16.restype = i
    return lib


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


def relative_error(got, ref) -> float:
    """max |got - ref| / max |ref| (the reference's measure, tests/test_nf4gemv.py:59-61)."""
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    return float(np.abs(got - ref).max()) / max(scale, 1e-6) if ref.size else 0.0


def ulp16(values, dt) -> "np.ndarray":
    """Spacing of the 16-bit output type at |values| (dt 0 = fp16, 1 = bf16)."""
    import numpy as np

    a = np.abs(np.asarray(values, dtype=np.float64))
    mant = 10 if dt == 0 else 7
    e = np.floor(np.log2(np.maximum(a, 1e-30)))
    e = np.maximum(e, -14 if dt == 0 else -126)
    return np.exp2(e - mant)


def beyond_rounding_error(got, ref, dt) -> float:
    """max(|got - ref| - ulp(ref)/2, 0) / max|ref|: the error of a 16-bit result
    against an unrounded fp64 reference, net of the half-ulp the output type's
    own rounding must cost. (bf16 keeps 8 significant bits, so that rounding
    alone is up to 2^-9 of each value - as large as the 2e-3 bar itself.)"""
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    excess = np.maximum(np.abs(got - ref) - 0.5 * ulp16(ref, dt), 0.0)
    return float(excess.max()) / max(float(np.abs(ref).max()), 1e-6)
