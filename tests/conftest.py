import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, "tests", "golden", "golden.npz")
SEED_BASE = 0x52504C00


def seed(cfg, stream):
    """Seed of input stream `stream` of config `cfg` (configs follow
    BASELINE.json; 90+ are fixture-only cases)."""
    return SEED_BASE + 16 * cfg + stream


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as g:
        return {k: g[k] for k in g.files}


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def rpl():
    import rpl_amd

    return rpl_amd.lib()


@pytest.fixture(scope="session")
def gpu(rpl):
    """The product library with an initialised gfx950 device (GPU tests)."""
    st = rpl.rplhip_init()
    if st != 0:
        pytest.fail(f"gfx950 device not usable: {rpl.rplhip_last_error().decode()}")
    return rpl


@pytest.fixture(autouse=True)
def _clean_last_error(request):
    """rpl_last_error() keeps the last failure of the thread: start every
    test that uses the library with a clean slate."""
    if "rpl" in request.fixturenames or "gpu" in request.fixturenames:
        request.getfixturevalue("rpl").rpl_clear_last_error()
    yield


def bits_equal(a, b):
    """Bit-level equality (NaN payloads and signed zeros included)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def gemm_err_ratio(C, A, B, C_ref):
    """max_ij |C - C_ref| / sum_k |a_ik b_kj| (float64), the fp32 GEMM
    parity metric: bounded by ~K*eps for any summation order."""
    denom = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    denom = np.maximum(denom, np.finfo(np.float64).tiny)
    return float(np.max(np.abs(C.astype(np.float64) - C_ref.astype(np.float64)) / denom))
