"""FP32 GEMM on f32 MFMA vs the oracle / reference golden vectors.

Tolerance (written here, as BASELINE.json's north star states it):
max_ij |C - C_ref| / sum_k |a_ik b_kj| <= 1e-5 * sqrt(K).
"""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal, seed
from gpu_util import fp32_tol, gemm_err_ratio, say, sgemm

pytestmark = pytest.mark.gpu


def op(X, t):
    return X.T if t else X


@pytest.mark.parametrize("name,ta,tb", [("nn", 0, 0), ("nt", 0, 1), ("tn", 1, 0), ("tt", 1, 1)])
def test_sgemm_golden(gpu, golden, name, ta, tb):
    A, B, C0 = golden[f"sgemm_{name}_A"], golden[f"sgemm_{name}_B"], golden[f"sgemm_{name}_C0"]
    M, N = C0.shape
    K = A.shape[0] if ta else A.shape[1]
    say("sgemm golden", name, M, N, K)
    out = sgemm(A, B, C0, M, N, K, 0.75, -0.5, ta, tb)
    assert gemm_err_ratio(out, op(A, ta), op(B, tb), golden[f"sgemm_{name}_C"], 0.75, -0.5, C0) <= fp32_tol(K)


# Products with K <= 256 and M*N*K <= 2^23 run on the VALU kernel in the
# reference's operation order (sequential fma over k, then
# fma(alpha, sum, beta*C)): bit-exact with the reference's golden vectors and
# the oracle, including the MLP's 4096x128x10 and 4096x10x128.
@pytest.mark.parametrize("name,ta,tb", [("nn", 0, 0), ("nt", 0, 1), ("tn", 1, 0), ("tt", 1, 1)])
def test_sgemm_small_golden_bit_exact(gpu, golden, name, ta, tb):
    A, B, C0 = golden[f"sgemm_{name}_A"], golden[f"sgemm_{name}_B"], golden[f"sgemm_{name}_C0"]
    M, N = C0.shape
    K = A.shape[0] if ta else A.shape[1]
    say("sgemm small golden bit-exact", name, M, N, K)
    assert bits_equal(sgemm(A, B, C0, M, N, K, 0.75, -0.5, ta, tb), golden[f"sgemm_{name}_C"])


@pytest.mark.parametrize("M,N,K", [(4096, 128, 10), (4096, 10, 128), (1, 1, 1), (3, 5, 7), (33, 17, 256),
                                   (200, 130, 1), (10, 128, 300)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_small_vs_oracle(gpu, orc, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 3 + N * 5 + K + 2 * ta + tb)
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    for alpha, beta in ((1.0, 0.0), (0.75, -0.5), (1.0, 1.0)):
        say("sgemm small", M, N, K, ta, tb, alpha, beta)
        out = sgemm(A, B, C0, M, N, K, alpha, beta, ta, tb)
        ref = orc.sgemm(A, B, C0, M, N, K, alpha, beta, bool(ta), bool(tb))
        if K <= 256:
            assert bits_equal(out, ref)
        else:  # (10, 128, 300): K past the single-pass bound (wave-split kernel, or VALU k slices)
            assert gemm_err_ratio(out, op(A, ta), op(B, tb), ref, alpha, beta, C0) <= fp32_tol(K)


@pytest.mark.parametrize("M,N,K,ld", [(64, 16, 130, 132), (64, 16, 128, 132), (1000, 1, 32, 36), (100, 64, 128, 128),
                                      (77, 3, 252, 256)])
def test_sgemm_small_padded_rows_bit_exact(gpu, orc, M, N, K, ld):
    # A as [M,K] and B as [N,K] with 16-byte aligned rows: K % 4 == 0 and
    # N <= 64 stage the block's rows in LDS (k_sgemm_valu_lds: N = 1, 16, 64,
    # ragged last blocks); (77, 3, 252) would need more than 64 KB of LDS and
    # K % 4 == 2 cannot stage, so both take 128-bit loads from memory (with
    # two scalar steps for K = 130); the fma chain is the reference's always.
    rng = np.random.default_rng(M + N + K)
    Abig = rng.uniform(-1, 1, (M, ld)).astype(np.float32)
    Bbig = rng.uniform(-1, 1, (N, ld)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    say("sgemm small padded rows", M, N, K, ld)
    out = sgemm(Abig, Bbig, C0, M, N, K, 0.75, -0.5, 0, 1, lda=ld, ldb=ld)
    ref = orc.sgemm(Abig[:, :K].copy(), Bbig[:, :K].copy(), C0, M, N, K, 0.75, -0.5, False, True)
    assert bits_equal(out, ref)


def test_sgemm_nan_in_c_propagates(gpu, golden):
    say("sgemm nan")
    out = sgemm(golden["sgemm_nan_A"], golden["sgemm_nan_A"], golden["sgemm_nan_C0"], 4, 4, 4, 1.0, 0.0)
    ref = golden["sgemm_nan_C"]
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    np.testing.assert_allclose(out[~np.isnan(ref)], ref[~np.isnan(ref)], rtol=1e-6)


def test_sgemm_split_k_nan_in_c(gpu):
    # tensor_gemm reads C even when beta == 0 (src/rpl_core.c:214): a NaN in C
    # survives the split-K reduction too.
    rng = np.random.default_rng(3)
    M, N, K = 8, 8, 1024
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = np.zeros((M, N), np.float32)
    C0[2, 3] = np.nan
    say("sgemm split-K nan")
    out = sgemm(A, B, C0, M, N, K, 1.0, 0.0)
    assert np.isnan(out[2, 3]) and np.isnan(out).sum() == 1
    ref = A.astype(np.float64) @ B.astype(np.float64)
    mask = ~np.isnan(out)
    assert np.max(np.abs(out[mask] - ref[mask]) / (np.abs(A) @ np.abs(B))[mask]) <= fp32_tol(K)


def test_sgemm_known_answers(gpu):
    # tests/full_system_check.py:33-37 and examples/gpu_test.c:106-128 (exact)
    say("sgemm known answers")
    eye = np.eye(128, dtype=np.float32)
    ones = np.ones((128, 128), np.float32)
    assert np.array_equal(sgemm(eye, ones, np.zeros_like(ones), 128, 128, 128), ones)
    o32 = np.ones((32, 32), np.float32)
    assert np.array_equal(sgemm(o32, np.eye(32, dtype=np.float32), np.zeros_like(o32), 32, 32, 32), o32)
    A = np.random.default_rng(1).standard_normal((256, 256)).astype(np.float32)
    assert np.array_equal(sgemm(A, np.eye(256, dtype=np.float32), np.zeros_like(A), 256, 256, 256), A)


# (17, 33, 2049) takes the split-K path of the 128 x 128 kernel (few tiles,
# long K, N % 4 != 0): partial tiles in a workspace, then
# C = alpha * sum + beta * C; (128, 784, 4096), (10, 128, 4096) and
# (512, 512, 512) the wave-split kernel.
SHAPES = [(1, 1, 1), (3, 5, 7), (127, 129, 65), (130, 7, 300), (64, 256, 32), (200, 130, 1), (17, 33, 2049),
          (256, 256, 0), (128, 784, 4096), (10, 128, 4096), (512, 512, 512)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_ragged_vs_oracle(gpu, orc, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 1000 + N * 10 + K + 7 * ta + 3 * tb)
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    say("sgemm ragged", M, N, K, ta, tb)
    out = sgemm(A, B, C0, M, N, K, 1.25, 0.5, ta, tb)
    ref = orc.sgemm(A, B, C0, M, N, K, 1.25, 0.5, bool(ta), bool(tb))
    assert gemm_err_ratio(out, op(A, ta), op(B, tb), ref, 1.25, 0.5, C0) <= fp32_tol(K)


# Small grids (a K split of the 128 x 128 tiles, or K > 256 with
# M*N*K <= 2^23) on the wave-split kernel, 128-bit shapes only: tiles of
# 16 / 32 / 64 rows x 64 columns, four waves per tile each over a quarter of
# the block's K range, K split over blocks when the tiles are few.  Shapes
# cover each tile height, a partial last 16-k step (K % 16 != 0), columns
# and rows past the matrix in edge tiles, no split / a few / 256 splits, the
# MLP's three products, and operands the kernel does not take (K % 4 != 0
# with a k-contiguous operand: the older paths).  A NaN in C stays where it
# is (C is read).
WS_SHAPES = [(4096, 128, 784), (4096, 128, 792), (128, 784, 4096), (10, 128, 4096), (12, 128, 4100),
             (36, 68, 1000), (1000, 100, 300), (512, 512, 512), (64, 64, 65536), (20, 8, 260), (16, 64, 1025)]


@pytest.mark.parametrize("M,N,K", WS_SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_wave_split_vs_float64(gpu, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 3 + K + 2 * ta + tb)
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    C0[M // 2, N // 3] = np.nan
    alpha, beta = 0.75, -0.5
    say("sgemm wave split", M, N, K, ta, tb)
    out = sgemm(A, B, C0, M, N, K, alpha, beta, ta, tb)
    assert np.isnan(out[M // 2, N // 3]) and np.isnan(out).sum() == 1
    opA, opB = op(A, ta).astype(np.float64), op(B, tb).astype(np.float64)
    ref = alpha * (opA @ opB) + beta * C0.astype(np.float64)
    ok = ~np.isnan(ref)
    assert gemm_err_ratio(np.where(ok, out, 0), op(A, ta), op(B, tb), np.where(ok, ref, 0), alpha, beta,
                          np.nan_to_num(C0)) <= fp32_tol(K)


def _ws_random_shapes(n, seed_):
    # Shapes the wave-split kernel takes: N % 4 == 0, M % 4 == 0 and K % 4 == 0
    # (so every transpose qualifies), K > 256, and either M*N*K <= 2^23 or
    # too few 128 x 128 tiles to fill the CUs.
    rng = np.random.default_rng(seed_)
    out = []
    while len(out) < n:
        M = 4 * int(rng.integers(1, 200))
        N = 4 * int(rng.integers(1, 100))
        K = 4 * int(rng.integers(65, 3000))
        tiles = -(-M // 128) * -(-N // 128)
        if M * N * K <= 1 << 23 or (tiles < 256 and K >= 256):
            out.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,ta,tb", _ws_random_shapes(24, 5))
def test_sgemm_wave_split_random(gpu, M, N, K, ta, tb):
    rng = np.random.default_rng(M + 3 * N + 7 * K + ta + 2 * tb)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    alpha, beta = 1.5, 0.25
    say("sgemm wave split random", M, N, K, ta, tb)
    out = sgemm(A, B, C0, M, N, K, alpha, beta, ta, tb)
    opA, opB = op(A, ta).astype(np.float64), op(B, tb).astype(np.float64)
    ref = alpha * (opA @ opB) + beta * C0.astype(np.float64)
    assert gemm_err_ratio(out, op(A, ta), op(B, tb), ref, alpha, beta, C0) <= fp32_tol(K)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_wave_split_leading_dimensions(gpu, ta, tb):
    # Sub-matrix views on the wave-split kernel: lda / ldb / ldc past the
    # extents (multiples of 4 floats), padding left untouched.
    rng = np.random.default_rng(20 + 2 * ta + tb)
    M, N, K = 64, 96, 1000
    pa, pb, pc = 12, 8, 4
    Abig = rng.uniform(-1, 1, (K, M + pa) if ta else (M, K + pa)).astype(np.float32)
    Bbig = rng.uniform(-1, 1, (N, K + pb) if tb else (K, N + pb)).astype(np.float32)
    Cbig = rng.uniform(-1, 1, (M, N + pc)).astype(np.float32)
    Cbig[5, 7] = np.nan
    lda, ldb, ldc = Abig.shape[1], Bbig.shape[1], N + pc
    say("sgemm wave split ld", ta, tb)
    out = sgemm(Abig, Bbig, Cbig, M, N, K, 0.75, -0.5, ta, tb, lda=lda, ldb=ldb, ldc=ldc)
    A = Abig[:, :M] if ta else Abig[:, :K]
    B = Bbig[:, :K] if tb else Bbig[:, :N]
    assert np.array_equal(out[:, N:], Cbig[:, N:])  # untouched padding
    assert np.isnan(out[5, 7]) and np.isnan(out[:, :N]).sum() == 1
    ref = 0.75 * (op(A, ta).astype(np.float64) @ op(B, tb).astype(np.float64)) - 0.5 * Cbig[:, :N].astype(np.float64)
    ok = ~np.isnan(ref)
    assert gemm_err_ratio(np.where(ok, out[:, :N], 0), op(A, ta), op(B, tb), np.where(ok, ref, 0), 0.75, -0.5,
                          np.nan_to_num(Cbig[:, :N])) <= fp32_tol(K)


def test_sgemm_leading_dimensions(gpu, orc):
    # Sub-matrix views: lda/ldb/ldc larger than the extents (gemm_optimized's lda/ldb/ldc).
    rng = np.random.default_rng(3)
    M, N, K = 70, 90, 110
    Abig = rng.uniform(-1, 1, (M, K + 13)).astype(np.float32)
    Bbig = rng.uniform(-1, 1, (K, N + 6)).astype(np.float32)
    Cbig = rng.uniform(-1, 1, (M, N + 3)).astype(np.float32)
    say("sgemm ld")
    out = sgemm(Abig, Bbig, Cbig, M, N, K, 1.0, 1.0, lda=K + 13, ldb=N + 6, ldc=N + 3)
    ref = Cbig.copy()
    ref[:, :N] = orc.sgemm(Abig[:, :K].copy(), Bbig[:, :N].copy(), Cbig[:, :N].copy(), M, N, K, 1.0, 1.0)
    assert np.array_equal(out[:, N:], Cbig[:, N:])  # untouched padding
    assert gemm_err_ratio(out[:, :N], Abig[:, :K], Bbig[:, :N], ref[:, :N], 1.0, 1.0, Cbig[:, :N]) <= fp32_tol(K)


def test_config0_512_vs_oracle(gpu, orc):
    n = 512
    A = rpl_amd.fill_uniform(n * n, seed(0, 0)).reshape(n, n)
    B = rpl_amd.fill_uniform(n * n, seed(0, 1)).reshape(n, n)
    say("config 0: sgemm 512^3")
    out = sgemm(A, B, np.zeros((n, n), np.float32), n, n, n)
    ref = orc.sgemm(A, B, np.zeros((n, n), np.float32), n, n, n)
    assert gemm_err_ratio(out, A, B, ref) <= fp32_tol(n)


def test_config4_8192_sampled_rows(gpu):
    n = 8192
    A = rpl_amd.fill_normal(n * n, seed(4, 0)).reshape(n, n)
    B = rpl_amd.fill_normal(n * n, seed(4, 1)).reshape(n, n)
    say("config 4: sgemm 8192^3")
    out = sgemm(A, B, np.zeros((n, n), np.float32), n, n, n)
    rows = np.random.default_rng(0).choice(n, 24, replace=False)
    ref = A[rows].astype(np.float64) @ B.astype(np.float64)
    denom = np.abs(A[rows].astype(np.float64)) @ np.abs(B.astype(np.float64))
    assert np.max(np.abs(out[rows] - ref) / denom) <= fp32_tol(n)
    # Size-independent property over every row: C @ x == A @ (B @ x).
    x = np.random.default_rng(1).standard_normal(n)
    lhs = out.astype(np.float64) @ x
    rhs = A.astype(np.float64) @ (B.astype(np.float64) @ x)
    scale = np.abs(A.astype(np.float64)) @ (np.abs(B.astype(np.float64)) @ np.abs(x))
    assert np.max(np.abs(lhs - rhs) / scale) <= fp32_tol(n)


# Grids with >= 2 tiles of 256 x 256 per CU take the direct-to-LDS kernel
# (k_sgemm_dma).  (5900, 5892, 1040): ragged M and N edges, 65 k-tiles (the
# unrolled steady-state loop plus a 5-tile tail); (6144, 6144, 48): only the
# tail loop.  All four transposes, alpha/beta, a NaN in C (C is always read).
@pytest.mark.parametrize("M,N,K", [(5900, 5892, 1040), (6144, 6144, 48)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_big_tile_paths(gpu, M, N, K, ta, tb):
    rng = np.random.default_rng(M + N + K + 2 * ta + tb)
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    C0[M // 2, N // 3] = np.nan
    alpha, beta = 0.75, -0.5
    say("sgemm big tile", M, N, K, ta, tb)
    out = sgemm(A, B, C0, M, N, K, alpha, beta, ta, tb)
    opA, opB = op(A, ta).astype(np.float64), op(B, tb).astype(np.float64)
    assert np.isnan(out[M // 2, N // 3]) and np.isnan(out).sum() == 1
    rows = np.unique(np.concatenate([[0, M - 1, M // 2], rng.choice(M, 12, replace=False)]))
    ref = alpha * (opA[rows] @ opB) + beta * C0[rows].astype(np.float64)
    denom = abs(alpha) * (np.abs(opA[rows]) @ np.abs(opB)) + abs(beta) * np.abs(C0[rows].astype(np.float64))
    ok = ~np.isnan(ref)
    assert np.max(np.abs(out[rows] - ref)[ok] / denom[ok]) <= fp32_tol(K)
    # Every row and column through C x = alpha A (B x) + beta C0 x (NaN column dropped).
    x = rng.standard_normal(N)
    x[N // 3] = 0.0
    c0 = np.nan_to_num(C0.astype(np.float64))
    o = np.nan_to_num(out.astype(np.float64))
    lhs = o @ x
    rhs = alpha * (opA @ (opB @ x)) + beta * (c0 @ x)
    scale = abs(alpha) * (np.abs(opA) @ (np.abs(opB) @ np.abs(x))) + abs(beta) * (np.abs(c0) @ np.abs(x))
    assert np.max(np.abs(lhs - rhs) / scale) <= fp32_tol(K)
    y = rng.standard_normal(M)
    y[M // 2] = 0.0
    lhs = y @ o
    rhs = alpha * ((y @ opA) @ opB) + beta * (y @ c0)
    scale = abs(alpha) * ((np.abs(y) @ np.abs(opA)) @ np.abs(opB)) + abs(beta) * (np.abs(y) @ np.abs(c0))
    assert np.max(np.abs(lhs - rhs) / scale) <= fp32_tol(K)


# ---------------------------------------------------- through include/rpl.h

def tensor_from(lib, arr, requires_grad=False):
    arr = np.ascontiguousarray(arr, np.float32)
    shape = (C.c_uint32 * arr.ndim)(*arr.shape)
    t = lib.tensor_create(arr.ndim, shape, requires_grad)
    C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def tensor_data(t, shape):
    return np.ctypeslib.as_array(t.contents.data, shape=(t.contents.size,)).copy().reshape(shape)


@pytest.mark.parametrize("resident", [False, True])
def test_tensor_gemm_api(gpu, orc, golden, resident):
    lib = gpu
    for name, ta, tb in (("nn", 0, 0), ("nt", 0, 1), ("tn", 1, 0), ("tt", 1, 1)):
        A, B, C0 = golden[f"sgemm_{name}_A"], golden[f"sgemm_{name}_B"], golden[f"sgemm_{name}_C0"]
        M, N = C0.shape
        K = A.shape[0] if ta else A.shape[1]
        tA, tB, tC = tensor_from(lib, A), tensor_from(lib, B), tensor_from(lib, C0)
        if resident:
            for t in (tA, tB, tC):
                lib.tensor_to_gpu(t)
            assert tC.contents.device == rpl_amd.DEVICE_GPU and tC.contents.gpu_buffer != 0
        say("tensor_gemm", name, "resident" if resident else "host")
        lib.tensor_gemm(tC, tA, tB, 0.75, -0.5, bool(ta), bool(tb))
        if resident:
            lib.tensor_from_gpu(tC)
        out = tensor_data(tC, (M, N))
        assert gemm_err_ratio(out, op(A, ta), op(B, tb), golden[f"sgemm_{name}_C"], 0.75, -0.5, C0) <= fp32_tol(K)
        for t in (tA, tB, tC):
            lib.tensor_free(t)


@pytest.mark.parametrize("resident", [False, True])
@pytest.mark.parametrize("name", ["mha_s5_d8", "mha_s8_d8", "mha_s3_d16"])
def test_tensor_gemm_3d_projection(gpu, golden, name, resident):
    """multi_head_attention_forward's projections (src/rpl_attention.c:175-177,
    232): tensor_gemm on [b,s,d] tensors with W [d,d] and trans_b takes
    M = b, K = s, N = d from shape[0..1].  Reference golden, bit-exact (K <= 256:
    the reference's operation order)."""
    lib = gpu
    A, W, want = golden[f"sgemm3d_{name}_A"], golden[f"sgemm3d_{name}_W"], golden[f"sgemm3d_{name}_C"]
    tA, tW, tC = tensor_from(lib, A), tensor_from(lib, W), tensor_from(lib, np.zeros(A.shape, np.float32))
    if resident:
        for t in (tA, tW, tC):
            lib.tensor_to_gpu(t)
    say("tensor_gemm 3-D", name, "resident" if resident else "host")
    lib.tensor_gemm(tC, tA, tW, 1.0, 0.0, False, True)
    if resident:
        lib.tensor_from_gpu(tC)
    assert not lib.rpl_last_error()
    assert bits_equal(tensor_data(tC, A.shape), want)
    for t in (tA, tW, tC):
        lib.tensor_free(t)


def test_tensor_gemm_out_of_bounds_refused(gpu):
    """Where the reference would read past a buffer (seq > d_model: N*K
    exceeds W's size) the call is refused and C is left untouched."""
    lib = gpu
    A = np.ones((2, 9, 8), np.float32)
    W = np.ones((8, 8), np.float32)
    C0 = np.full((2, 9, 8), 3.0, np.float32)
    tA, tW, tC = tensor_from(lib, A), tensor_from(lib, W), tensor_from(lib, C0)
    say("tensor_gemm out of bounds")
    lib.tensor_gemm(tC, tA, tW, 1.0, 0.0, False, True)
    assert b"out of bounds" in lib.rpl_last_error()
    assert bits_equal(tensor_data(tC, C0.shape), C0)
    for t in (tA, tW, tC):
        lib.tensor_free(t)


def test_tensor_matmul_and_matmul_gpu(gpu, orc):
    lib = gpu
    rng = np.random.default_rng(8)
    A = rng.standard_normal((100, 60)).astype(np.float32)
    B = rng.standard_normal((60, 80)).astype(np.float32)
    tA, tB = tensor_from(lib, A), tensor_from(lib, B)
    say("tensor_matmul")
    out = lib.tensor_matmul(tA, tB)
    ref = orc.sgemm(A, B, np.zeros((100, 80), np.float32), 100, 80, 60)
    assert gemm_err_ratio(tensor_data(out, (100, 80)), A, B, ref) <= fp32_tol(60)
    tC = tensor_from(lib, np.zeros((100, 80), np.float32))
    say("tensor_matmul_gpu")
    lib.tensor_matmul_gpu(tC, tA, tB)
    lib.tensor_from_gpu(tC)
    assert gemm_err_ratio(tensor_data(tC, (100, 80)), A, B, ref) <= fp32_tol(60)
    for t in (tA, tB, tC, out):
        lib.tensor_free(t)


def test_parallel_gemm_optimized(gpu, orc, golden):
    lib = gpu
    fp = C.POINTER(C.c_float)
    A, B, C0 = golden["gemmopt_A"], golden["gemmopt_B"], golden["gemmopt_C0"].copy()
    say("parallel_gemm_optimized golden")
    lib.parallel_gemm_optimized(A.ctypes.data_as(fp), B.ctypes.data_as(fp), C0.ctypes.data_as(fp), 8, 4, 16)
    assert gemm_err_ratio(C0, A, B, golden["gemmopt_C"], 1.0, 1.0, golden["gemmopt_C0"]) <= fp32_tol(16)
    rng = np.random.default_rng(4)
    M, N, K = 300, 257, 513
    A = rng.uniform(0, 1, (M, K)).astype(np.float32)
    B = rng.uniform(0, 1, (K, N)).astype(np.float32)
    C1 = rng.uniform(0, 1, (M, N)).astype(np.float32)
    out = C1.copy()
    say("parallel_gemm_optimized random")
    lib.parallel_gemm_optimized(A.ctypes.data_as(fp), B.ctypes.data_as(fp), out.ctypes.data_as(fp), M, N, K)
    ref = orc.sgemm(A, B, C1, M, N, K, 1.0, 1.0)
    assert gemm_err_ratio(out, A, B, ref, 1.0, 1.0, C1) <= fp32_tol(K)


def test_workspace_reuse_across_streams(gpu):
    # Split-K GEMMs keep their partial tiles in cached workspace blocks; a
    # block is reused only in the stream order of its last user.  Queue
    # calls of two shapes on two streams without synchronising in between,
    # destroy one stream half way, and check every result.
    lib = rpl_amd.lib()
    from rpl_amd import DeviceBuffer, check
    rng = np.random.default_rng(11)
    streams = []
    for _ in range(3):
        s = C.c_void_p()
        check(lib.rplhip_stream_create(C.byref(s)), "stream_create")
        streams.append(s)
    jobs = []
    for i in range(12):
        M, N, K = ((10, 128, 4096), (128, 784, 4096), (17, 33, 2049))[i % 3]
        A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        dA, dB, dC = DeviceBuffer.from_array(A), DeviceBuffer.from_array(B), DeviceBuffer.from_array(
            np.zeros((M, N), np.float32))
        s = streams[2] if i >= 6 and i % 2 == 0 else streams[i % 2]
        check(lib.rplhip_sgemm(0, 0, M, N, K, 1.0, dA.ptr, K, dB.ptr, N, 0.0, dC.ptr, N, s), "sgemm")
        jobs.append((A, B, dA, dB, dC, M, N, K))
        if i == 5:
            check(lib.rplhip_stream_destroy(streams[0]), "stream_destroy")
            streams[0] = C.c_void_p()
            check(lib.rplhip_stream_create(C.byref(streams[0])), "stream_create")
    say("workspace reuse across streams", len(jobs))
    for s in streams:
        check(lib.rplhip_stream_synchronize(s), "stream_synchronize")
    for A, B, dA, dB, dC, M, N, K in jobs:
        out = dC.to_array(np.float32, (M, N))
        ref = A.astype(np.float64) @ B.astype(np.float64)
        assert np.max(np.abs(out - ref) / (np.abs(A) @ np.abs(B))) <= fp32_tol(K)
    for s in streams:
        check(lib.rplhip_stream_destroy(s), "stream_destroy")


# rplhip_sgemm_batched: one launch for `batch` GEMMs of one shape (the
# attention products).  read_c = 0 writes C without reading it (C starts as
# NaN and none may survive); read_c = 1 is alpha*AB + beta*C per batch.
@pytest.mark.parametrize("M,N,K,ta,tb,batch", [(64, 64, 32, 0, 1, 3), (200, 130, 48, 0, 0, 5), (33, 17, 9, 1, 0, 2),
                                               (128, 256, 64, 1, 1, 7), (130, 72, 300, 0, 1, 1)])
def test_sgemm_batched(gpu, M, N, K, ta, tb, batch):
    from gpu_util import down, empty, up
    lib = gpu
    rng = np.random.default_rng(M + N + K + batch)
    A = rng.uniform(-1, 1, (batch,) + ((K, M) if ta else (M, K))).astype(np.float32)
    B = rng.uniform(-1, 1, (batch,) + ((N, K) if tb else (K, N))).astype(np.float32)
    C0 = rng.uniform(-1, 1, (batch, M, N)).astype(np.float32)
    lda, ldb = (M if ta else K), (K if tb else N)
    dA, dB = up(A), up(B)
    for read_c in (0, 1):
        dC = up(np.full((batch, M, N), np.nan, np.float32) if read_c == 0 else C0)
        say("sgemm batched", M, N, K, ta, tb, batch, read_c)
        rpl_amd.check(lib.rplhip_sgemm_batched(ta, tb, M, N, K, 1.25, dA.ptr, lda, M * K, dB.ptr, ldb, N * K, 0.5,
                                               dC.ptr, N, M * N, batch, read_c, None))
        got = down(dC, np.float32, (batch, M, N))
        assert np.isfinite(got).all()
        for z in range(batch):
            a, b = op(A[z], ta), op(B[z], tb)
            ref = 1.25 * (a.astype(np.float64) @ b.astype(np.float64)) + (0.5 * C0[z] if read_c else 0.0)
            assert gemm_err_ratio(got[z], a, b, ref, 1.25, 0.5 if read_c else 0.0,
                                  C0[z] if read_c else None) <= fp32_tol(K)
