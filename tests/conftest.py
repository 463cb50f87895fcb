import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "nki-kernel-lab_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import pytest  # noqa: E402

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libnkilab_hip.so")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def rel_err(a, b):
    """max|a - b| / max|b| in float64: the reference's tolerance metric."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-12))


def bf16_ulp(x):
    """Spacing of bfloat16 numbers at |x| (2^-7 relative, 8 significand bits)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_within_bf16_ulps(out, ref, ulps=1.0, floor=0.0):
    """Every element of a bf16 result within `ulps` bf16 ulps (of the reference
    value) of the reference, plus an absolute floor for values near zero."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = ulps * bf16_ulp(ref) + floor
    bad = np.abs(out - ref) > bound
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements beyond {ulps} bf16 ulp; worst "
                           f"{np.abs(out - ref).max():.3g} at ref {ref.flat[np.argmax(np.abs(out - ref))]:.4g}")


def load_golden(name):
    return dict(np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False))


@pytest.fixture
def flash_cfg():
    """Force the bf16 attention kernel / schedule / block / block start cost for
    one test (nkl_flash_attn_configure), restoring the automatic choice after."""
    from nkilab import _lib

    yield _lib.flash_configure
    _lib.flash_configure()
    _lib.flash_configure_polls()
