"""Seeded randomized parity sweep across the dispatch paths: shapes drawn
from small/ragged/aligned classes (every kernel choice the dispatchers make
below the big-tile sizes: decode, skinny, register-staged, 256 x 128 and
256 x 256 direct-to-LDS tiles, split-K, transposed or in-place B), random
scales, zero points and transposes, against the oracle.  Bars as elsewhere:
bit-exact for int8 results and the fused fp32 dequant, 1e-5 * sqrt(K) of
sum |a b| for fp32 GEMMs."""
import numpy as np
import pytest

from gpu_util import fp32_tol, gemm_err_ratio, gemm_int8, linear_int8_dequant, say, sgemm

pytestmark = pytest.mark.gpu

SWEEP_SEED = 0x5EED


def _dims(rng, i):
    # A third each: tiny/ragged, 64/128-aligned mid-size, M <= 16 skinny.
    c = i % 3
    if c == 0:
        return int(rng.integers(1, 97)), int(rng.integers(1, 130)), int(rng.integers(1, 260))
    if c == 1:
        return int(rng.integers(1, 9)) * 64, int(rng.integers(1, 9)) * 64, int(rng.integers(1, 9)) * 128
    return int(rng.integers(1, 17)), int(rng.integers(1, 300)), int(rng.integers(1, 5)) * 512


@pytest.mark.parametrize("i", range(24))
def test_sweep_gemm_int8(gpu, orc, i):
    rng = np.random.default_rng(SWEEP_SEED + i)
    M, N, K = _dims(rng, i)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    sa, sb = float(rng.uniform(1e-3, 0.1)), float(rng.uniform(1e-3, 0.1))
    sc = float([1.0, 0.5, rng.uniform(0.1, 3.0)][i % 3])
    za, zb = (0, 0) if i % 2 else (int(rng.integers(-20, 20)), int(rng.integers(-20, 20)))
    say("sweep gemm_int8", i, M, N, K, sa, sb, sc, za, zb)
    got = gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb)
    assert np.array_equal(got, orc.gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb))


@pytest.mark.parametrize("i", range(24))
def test_sweep_linear_int8_dequant(gpu, orc, i):
    rng = np.random.default_rng(SWEEP_SEED + 100 + i)
    M, N, K = _dims(rng, i)
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    x_row, w_col = bool(i % 2), bool((i // 2) % 2)
    sx = rng.uniform(1e-3, 0.05, M if x_row else 1).astype(np.float32)
    sw = rng.uniform(1e-3, 0.05, N if w_col else 1).astype(np.float32)
    say("sweep linear_int8_dequant", i, M, N, K, x_row, w_col)
    got = linear_int8_dequant(x, sx, int(x_row), w, sw, int(w_col), M, K, N)
    acc = orc.linear_int8(x, w, None, M, K, N)
    assert np.array_equal(got.view(np.uint32), orc.dequant_acc(acc, sx, x_row, sw, w_col).view(np.uint32))


@pytest.mark.parametrize("i", range(24))
def test_sweep_sgemm(gpu, orc, i):
    rng = np.random.default_rng(SWEEP_SEED + 200 + i)
    M, N, K = _dims(rng, i)
    ta, tb = i % 2, (i // 2) % 2
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    alpha, beta = float(rng.uniform(-2, 2)), float([0.0, 1.0, rng.uniform(-1, 1)][i % 3])
    say("sweep sgemm", i, M, N, K, ta, tb, alpha, beta)
    out = sgemm(A, B, C0, M, N, K, alpha, beta, ta, tb)
    ref = orc.sgemm(A, B, C0, M, N, K, alpha, beta, bool(ta), bool(tb))
    a = A.T if ta else A
    b = B.T if tb else B
    assert gemm_err_ratio(out, a, b, ref, alpha, beta, C0) <= fp32_tol(K)
