"""INT8 GEMMs on i8 MFMA vs the oracle and the reference golden vectors.
Bar: bit-exact (int32 accumulators, requantized int32, fused fp32 dequant)."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal, seed
from gpu_util import down, empty, gemm_int8, linear_int8, linear_int8_dequant, say, up

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", ["zp", "unit", "k1041", "overflow", "sc0", "tiny"])
def test_gemm_int8_golden(gpu, golden, case):
    A, B = golden[f"i8_{case}_A"], golden[f"i8_{case}_B"]
    sa, sb, sc = (float(v) for v in golden[f"i8_{case}_params"])
    za, zb = (int(v) for v in golden[f"i8_{case}_zp"])
    M, K = A.shape
    N = B.shape[1]
    say("gemm_int8 golden", case, M, N, K)
    assert bits_equal(gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb), golden[f"i8_{case}_C"])


def test_gemm_int8_rpl_api(gpu, golden):
    # include/rpl.h gemm_int8 on host pointers (staged through the device).
    i8p, i32p = C.POINTER(C.c_int8), C.POINTER(C.c_int32)
    A, B = golden["i8_zp_A"], golden["i8_zp_B"]
    M, K = A.shape
    N = B.shape[1]
    out = np.zeros((M, N), np.int32)
    say("rpl.h gemm_int8")
    gpu.gemm_int8(A.ctypes.data_as(i8p), B.ctypes.data_as(i8p), out.ctypes.data_as(i32p), M, N, K, 0.01, 0.02, 0.5,
                  3, -5)
    assert bits_equal(out, golden["i8_zp_C"])


# K and N multiples of 128 (256x256x512, 200x384x256, 16x1280x896,
# 3x128x8192) transpose B with whole 128x128 tiles (k_transpose_i8_tr); the
# others take the bounds-checked transpose.
SHAPES = [(1, 1, 1), (4, 9, 16), (16, 100, 64), (17, 31, 300), (129, 127, 129), (256, 256, 512), (64, 8, 1000),
          (5, 300, 4096), (200, 384, 256), (16, 1280, 896), (3, 128, 8192)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_int8_ragged_vs_oracle(gpu, orc, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    for (sa, sb, sc, za, zb) in ((1.0, 1.0, 1.0, 0, 0), (0.013, 0.7, 0.29, -2, 9)):
        say("gemm_int8 ragged", M, N, K, za, zb)
        got = gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb)
        assert bits_equal(got, orc.gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb))


@pytest.mark.parametrize("name", ["bias", "nobias", "m1"])
def test_linear_int8_golden(gpu, golden, name):
    x, w = golden[f"lin8_{name}_x"], golden[f"lin8_{name}_w"]
    bias = golden.get(f"lin8_{name}_bias")
    M, K = x.shape
    N = w.shape[0]
    say("linear_int8 golden", name)
    assert bits_equal(linear_int8(x, w, bias, M, K, N), golden[f"lin8_{name}_out"])


@pytest.mark.parametrize("M,K,N", [(1, 64, 33), (3, 67, 40), (4, 8192, 257), (16, 1000, 64), (17, 512, 129),
                                   (100, 4096, 96), (300, 48, 512)])
def test_linear_int8_vs_oracle(gpu, orc, M, K, N):
    rng = np.random.default_rng(M + K + N)
    x = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    b = rng.integers(-128, 128, N, dtype=np.int8)
    say("linear_int8", M, K, N)
    assert bits_equal(linear_int8(x, w, b, M, K, N), orc.linear_int8(x, w, b, M, K, N))
    assert bits_equal(linear_int8(x, w, None, M, K, N), orc.linear_int8(x, w, None, M, K, N))


# Small grids with short K take one wave per 32 x 32 tile (k_gemm_i8_small):
# ragged M and N, K % 32 == 16 (a last half step whose upper k-half is zero;
# K = 16 is that step alone), fewer k-steps than the 8 in flight, and the
# K = 2048 limit; raw with and without bias, requant with zero points on both
# sides (B's column sums from the transposed copy), and both dequant entry
# points, all bit-exact against the oracle.
@pytest.mark.parametrize("M,N,K", [(33, 65, 16), (96, 80, 48), (17, 40, 160), (100, 200, 1040), (257, 31, 2048),
                                   (512, 512, 512)])
def test_small_grid_int8_vs_oracle(gpu, orc, M, N, K):
    rng = np.random.default_rng(M * 5 + N + K)
    x = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    b = rng.integers(-128, 128, N, dtype=np.int8)
    say("small-grid linear_int8", M, N, K)
    assert bits_equal(linear_int8(x, w, b, M, K, N), orc.linear_int8(x, w, b, M, K, N))
    acc = orc.linear_int8(x, w, None, M, K, N)
    assert bits_equal(linear_int8(x, w, None, M, K, N), acc)
    B = np.ascontiguousarray(w.T)
    for (sa, sb, sc, za, zb) in ((1.0, 1.0, 1.0, 0, 0), (0.013, 0.7, 0.29, -3, 11)):
        say("small-grid gemm_int8", M, N, K, za, zb)
        assert bits_equal(gemm_int8(x, B, M, N, K, sa, sb, sc, za, zb), orc.gemm_int8(x, B, M, N, K, sa, sb, sc, za, zb))
    sx = rng.random(M).astype(np.float32) * 0.01
    sw = rng.random(N).astype(np.float32) * 0.02
    say("small-grid linear_int8_dequant", M, N, K)
    assert bits_equal(linear_int8_dequant(x, sx, True, w, sw, True, M, K, N), orc.dequant_acc(acc, sx, True, sw, True))
    lib = gpu
    dx, dB, dsa, dsw, dY = up(x), up(B), up(sx[:1]), up(sw), empty((M, N), np.float32)
    say("small-grid gemm_int8_dequant", M, N, K)
    rpl_amd.check(lib.rplhip_gemm_int8_dequant(dx.ptr, dsa.ptr, 0, dB.ptr, dsw.ptr, 1, dY.ptr, M, N, K, None))
    assert bits_equal(down(dY, np.float32, (M, N)), orc.dequant_acc(acc, sx[:1], False, sw, True))


# K = 0: every accumulator is the empty sum, so the outputs are the epilogue
# of 0 (requant of 0, sc = 0 -> 0/0 -> INT32_MIN, bias alone, 0 * scales).
# 4096 x 4096 is a grid the big-tile kernels would otherwise take.
@pytest.mark.parametrize("M,N", [(1, 7), (3, 5), (17, 40), (4096, 4096)])
def test_int8_k0_vs_oracle(gpu, orc, M, N):
    rng = np.random.default_rng(M + N)
    A, B, W = np.zeros((M, 0), np.int8), np.zeros((0, N), np.int8), np.zeros((N, 0), np.int8)
    for (sa, sb, sc, za, zb) in ((1.0, 1.0, 1.0, 0, 0), (0.013, 0.7, 0.29, -2, 9), (0.5, 0.25, 0.0, 0, 0),
                                 (0.5, 0.25, 0.125, 0, 0)):
        say("gemm_int8 K=0", M, N, sa, sb, sc, za, zb)
        assert bits_equal(gemm_int8(A, B, M, N, 0, sa, sb, sc, za, zb), orc.gemm_int8(A, B, M, N, 0, sa, sb, sc, za, zb))
    bias = rng.integers(-128, 128, N, dtype=np.int8)
    for b in (bias, None):
        say("linear_int8 K=0", M, N, b is not None)
        assert bits_equal(linear_int8(A, W, b, M, 0, N), orc.linear_int8(A, W, b, M, 0, N))
    sx = rng.random(M).astype(np.float32) * 0.01
    sw = rng.random(N).astype(np.float32) * 0.02
    say("linear_int8_dequant K=0", M, N)
    want = orc.dequant_acc(np.zeros((M, N), np.int32), sx, True, sw, True)
    assert bits_equal(linear_int8_dequant(A, sx, True, W, sw, True, M, 0, N), want)
    lib = rpl_amd.lib()
    dA, dB, dsa, dsb, dY = up(A), up(B), up(sx), up(sw), empty((M, N), np.float32)
    say("gemm_int8_dequant K=0", M, N)
    rpl_amd.check(lib.rplhip_gemm_int8_dequant(dA.ptr, dsa.ptr, 1, dB.ptr, dsb.ptr, 1, dY.ptr, M, N, 0, None))
    assert bits_equal(down(dY, np.float32, (M, N)), want)


@pytest.mark.parametrize("M,K,N", [(1, 256, 48), (16, 4096, 130), (77, 320, 200)])
def test_linear_int8_dequant_vs_oracle(gpu, orc, M, K, N):
    rng = np.random.default_rng(K)
    x = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sx = rng.random(M).astype(np.float32) * 0.01
    sw = rng.random(N).astype(np.float32) * 0.02
    acc = orc.linear_int8(x, w, None, M, K, N)
    for xr, wr in ((True, True), (False, False), (True, False)):
        say("linear_int8_dequant", M, K, N, xr, wr)
        got = linear_int8_dequant(x, sx if xr else sx[:1], xr, w, sw if wr else sw[:1], wr, M, K, N)
        assert bits_equal(got, orc.dequant_acc(acc, sx if xr else sx[:1], xr, sw if wr else sw[:1], wr))


def test_gemm_int8_dequant_vs_oracle(gpu, orc):
    lib = gpu
    rng = np.random.default_rng(31)
    M, N, K = 70, 90, 200
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    sa = np.float32([0.02])
    sb = rng.random(N).astype(np.float32)
    dA, dB, dsa, dsb, dY = up(A), up(B), up(sa), up(sb), empty((M, N), np.float32)
    say("gemm_int8_dequant")
    rpl_amd.check(lib.rplhip_gemm_int8_dequant(dA.ptr, dsa.ptr, 0, dB.ptr, dsb.ptr, 1, dY.ptr, M, N, K, None))
    acc = orc.gemm_int8(A, B, M, N, K)
    assert bits_equal(down(dY, np.float32, (M, N)), orc.dequant_acc(acc, sa, False, sb, True))


def test_config1_int8_512(gpu, golden):
    """Config 1: N(0,1) -> per-tensor symmetric quantize -> int32 GEMM, all on the device."""
    import hashlib

    lib = gpu
    n = 512
    A = rpl_amd.fill_normal(n * n, seed(1, 0))
    B = rpl_amd.fill_normal(n * n, seed(1, 1))
    dA, dB = up(A), up(B)
    qA, qB, sA, sB = empty(n * n, np.int8), empty(n * n, np.int8), empty(1, np.float32), empty(1, np.float32)
    say("config 1: quantize + gemm_int8 512^3")
    rpl_amd.check(lib.rplhip_quantize_symmetric(dA.ptr, n * n, qA.ptr, sA.ptr, None))
    rpl_amd.check(lib.rplhip_quantize_symmetric(dB.ptr, n * n, qB.ptr, sB.ptr, None))
    acc = empty((n, n), np.int32)
    rpl_amd.check(lib.rplhip_gemm_int8(qA.ptr, qB.ptr, acc.ptr, n, n, n, 1.0, 1.0, 1.0, 0, 0, None))
    scales = np.concatenate([down(sA, np.float32, (1,)), down(sB, np.float32, (1,))])
    assert bits_equal(scales, golden["cfg1_scales"])
    h = lambda a: hashlib.sha256(a.tobytes()).hexdigest().encode()  # noqa: E731
    assert h(down(qA, np.int8, (n * n,))) == golden["cfg1_qA_sha"].tobytes()
    assert h(down(qB, np.int8, (n * n,))) == golden["cfg1_qB_sha"].tobytes()
    assert h(down(acc, np.int32, (n, n))) == golden["cfg1_acc_sha"].tobytes()


@pytest.mark.parametrize("N", [4096, 11008])
def test_config3_transformer_linear(gpu, orc, N):
    """Config 3: X [2048,4096] per-token, W [N,4096] per-channel, fused dequant."""
    lib = gpu
    M, K = 2048, 4096
    X = rpl_amd.fill_normal(M * K, seed(3, 0)).reshape(M, K)
    W = rpl_amd.fill_normal(N * K, seed(3, 1), 0.0, 0.02).reshape(N, K)
    dX, dW = up(X), up(W)
    qX, qW = empty((M, K), np.int8), empty((N, K), np.int8)
    sX, sW = empty(M, np.float32), empty(N, np.float32)
    say("config 3: per-token / per-channel quantize", N)
    rpl_amd.check(lib.rplhip_quantize_per_channel(dX.ptr, M, K, qX.ptr, sX.ptr, None))
    rpl_amd.check(lib.rplhip_quantize_per_channel(dW.ptr, N, K, qW.ptr, sW.ptr, None))
    qx, sx = down(qX, np.int8, (M, K)), down(sX, np.float32, (M,))
    qw, sw = down(qW, np.int8, (N, K)), down(sW, np.float32, (N,))
    oqx, osx = orc.quantize_per_channel(X, M)
    oqw, osw = orc.quantize_per_channel(W, N)
    assert bits_equal(qx, oqx) and bits_equal(sx, osx) and bits_equal(qw, oqw) and bits_equal(sw, osw)
    Y = empty((M, N), np.float32)
    say("config 3: linear_int8_dequant", M, K, N)
    rpl_amd.check(lib.rplhip_linear_int8_dequant(qX.ptr, sX.ptr, 1, qW.ptr, sW.ptr, 1, Y.ptr, M, K, N, None))
    y = down(Y, np.float32, (M, N))
    rows = np.sort(np.random.default_rng(N).choice(M, 16, replace=False))
    acc_rows = orc.linear_int8(np.ascontiguousarray(qx[rows]), qw, None, len(rows), K, N)
    assert bits_equal(y[rows], orc.dequant_acc(acc_rows, sx[rows], True, sw, True))
    # Every row: the int32 path checked by an exact integer identity.
    acc = empty((M, N), np.int32)
    rpl_amd.check(lib.rplhip_linear_int8(qX.ptr, qW.ptr, None, acc.ptr, M, K, N, None))
    a = down(acc, np.int32, (M, N)).astype(np.int64)
    assert np.array_equal(a.sum(1), qx.astype(np.int64) @ qw.astype(np.int64).sum(0))
    assert np.array_equal(a.sum(0), qw.astype(np.int64) @ qx.astype(np.int64).sum(0))
    assert bits_equal(y, ((a.astype(np.int32).astype(np.float32) * sx[:, None]) * sw[None, :]))


@pytest.mark.parametrize("M", [1, 4, 16])
def test_config4_skinny(gpu, orc, M):
    """Config 4 skinny: M in {1,4,16}, K = N = 8192, per-channel W."""
    lib = gpu
    K = N = 8192
    X = rpl_amd.fill_normal(M * K, seed(4, 2)).reshape(M, K)
    W = rpl_amd.fill_normal(N * K, seed(4, 3)).reshape(N, K)
    qx, sx = orc.quantize_symmetric(X)
    qw, sw = orc.quantize_per_channel(W, N)
    say("config 4 skinny linear_int8", M)
    got = linear_int8(qx.reshape(M, K), qw, None, M, K, N)
    ref = orc.linear_int8(qx.reshape(M, K), qw, None, M, K, N)
    assert bits_equal(got, ref)
    say("config 4 skinny dequant", M)
    y = linear_int8_dequant(qx.reshape(M, K), np.float32([sx]), False, qw, sw, True, M, K, N)
    assert bits_equal(y, orc.dequant_acc(ref, np.float32([sx]), False, sw, True))


def test_config4_int8_8192(gpu, orc):
    """Config 4: 8192^3 per-tensor INT8 (gemm_int8 layout)."""
    lib = gpu
    n = 8192
    A = rpl_amd.fill_normal(n * n, seed(4, 0))
    B = rpl_amd.fill_normal(n * n, seed(4, 1))
    dA, dB = up(A), up(B)
    qA, qB, sA, sB = empty(n * n, np.int8), empty(n * n, np.int8), empty(1, np.float32), empty(1, np.float32)
    say("config 4: quantize 8192^2 x2")
    rpl_amd.check(lib.rplhip_quantize_symmetric(dA.ptr, n * n, qA.ptr, sA.ptr, None))
    rpl_amd.check(lib.rplhip_quantize_symmetric(dB.ptr, n * n, qB.ptr, sB.ptr, None))
    qa, qb = down(qA, np.int8, (n, n)), down(qB, np.int8, (n, n))
    oqa, osa = orc.quantize_symmetric(A)
    assert bits_equal(qa.reshape(-1), oqa) and bits_equal(down(sA, np.float32, (1,)), np.float32([osa]))
    del dA, dB, A, B
    acc = empty((n, n), np.int32)
    say("config 4: gemm_int8 8192^3")
    rpl_amd.check(lib.rplhip_gemm_int8(qA.ptr, qB.ptr, acc.ptr, n, n, n, 1.0, 1.0, 1.0, 0, 0, None))
    a = down(acc, np.int32, (n, n))
    rows = np.sort(np.random.default_rng(5).choice(n, 4, replace=False))
    ref_rows = orc.gemm_int8(np.ascontiguousarray(qa[rows]), qb, len(rows), n, n)
    assert bits_equal(a[rows], ref_rows)
    a64 = a.astype(np.int64)
    assert np.abs(a64).max() < 2 ** 24  # exact through the float requant with unit scales
    assert np.array_equal(a64.sum(1), qa.astype(np.int64) @ qb.astype(np.int64).sum(1))
    assert np.array_equal(a64.sum(0), qb.astype(np.int64).T @ qa.astype(np.int64).sum(0))


def _requant_f32(acc, sa, sb, sc):
    """x86((int32)roundf(((float)acc * sa) * sb / sc)) in numpy float32 (IEEE,
    one rounding per operation, as the reference at ops_extended.c:119)."""
    with np.errstate(all="ignore"):
        x = ((acc.astype(np.float32) * np.float32(sa)) * np.float32(sb)) / np.float32(sc)
        t = np.trunc(x)
        r = np.where(np.abs(x - t) >= np.float32(0.5), t + np.sign(x), t)  # roundf: ties away from zero
        ok = (r >= -2.0 ** 31) & (r < 2.0 ** 31)
    out = np.full(acc.shape, np.iinfo(np.int32).min, np.int32)
    out[ok] = r[ok].astype(np.int64).astype(np.int32)
    return out


# Shapes with >= 2 tiles of 256 x 256 per CU take the direct-to-LDS kernel
# (k_gemm_i8_nt_dma); K = 448 and 832 run its steady-state loop and tails of
# 3 and 5 tiles.  The first two shapes have ragged edges in M and N, so both
# the bounds-checked epilogue (edge tiles) and the unchecked buffer-store
# epilogue (interior tiles) run.  gemm_int8 and gemm_int8_dequant read B
# [K,N] in place when N % 16 == 0 (5888, 6144, 4400; at N = 4400 the last
# tile holds 48 columns and the chunks past them are clamped), and transpose
# it first otherwise (5900, 3000).  (1800, 3000, 448) has too few 256 x 256
# tiles and takes 256 x 128 ones (192 of them), with ragged M and N edges.
# K % 128 == 0 (896, 256, 128) copies A two k-steps at a time
# (k_gemm_i8_pairs): K = 896 runs three 4-k-step rounds of its loop and the
# 2-k-step remainder (with the copies past the end re-loading the last
# tile), K = 256 one round, K = 128 only the remainder.
# (4096, 3072, 128) is one k-step pair on the pairs kernel, (4096, 4096, 64)
# a single k-step on the per-k-step kernel.
# (3830, 5104 | 5110, 1024): 300 big tiles (two rounds, the second mostly
# idle) on the pairs kernel, 16 k-steps each, ragged M and N (5104: B [K,N]
# read in place by gemm_int8; 5110: through the transposed copy).
# K % 16 == 0 but K % 64 != 0 with at least two 256 x 256 tiles per CU
# (6144 x 6144: 576 tiles, 4096 x 8192: 512) takes the register-staged
# 256 x 256 kernel (k_gemm_i8_nt<CfgBig>): K = 848 is 13 whole 64-k tiles and
# a last tile holding 16 k-bytes (the rest zero-filled), K = 592 9 and the
# same; gemm_int8 reaches it through the transposed copy of B.
# (1800, 3000, K % 128 == 0) runs the 256 x 128 pairs kernel
# (k_gemm_i8_pairs_n128: three A pair slots, three B) with ragged M and N:
# K = 128 is one pair (every later copy clamped to it), 256 two, 384 one
# 4-k-step round and the remainder, 1152 four rounds and the remainder.
BIG = [(5890, 5900, 832), (5890, 5888, 832), (6144, 6144, 448), (1800, 3000, 448), (2900, 4400, 448),
       (5890, 5888, 896), (5890, 5900, 896), (2900, 4400, 256), (4096, 3072, 128), (4096, 4096, 64),
       (6144, 6144, 848), (4096, 8192, 592), (3830, 5104, 1024), (3830, 5110, 1024),
       (1800, 3000, 128), (1800, 3000, 256), (1800, 3000, 384), (1800, 3000, 1152)]


@pytest.mark.parametrize("M,N,K", BIG)
def test_big_tile_int8_paths(gpu, orc, M, N, K):
    lib = gpu
    rng = np.random.default_rng(M + K)
    A = np.clip(np.rint(rng.normal(0, 24, (M, K))), -127, 127).astype(np.int8)
    Bt = np.clip(np.rint(rng.normal(0, 24, (N, K))), -127, 127).astype(np.int8)
    B = np.ascontiguousarray(Bt.T)
    dA, dB, dBt = up(A), up(B), up(Bt)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(N).choice(M, 6, replace=False)]))
    # linear_int8 (raw int32): sampled rows vs the oracle, every row and column by exact sums.
    acc_d = empty((M, N), np.int32)
    say("big-tile linear_int8", M, N, K)
    rpl_amd.check(lib.rplhip_linear_int8(dA.ptr, dBt.ptr, None, acc_d.ptr, M, K, N, None))
    acc = down(acc_d, np.int32, (M, N))
    assert bits_equal(acc[rows], orc.linear_int8(np.ascontiguousarray(A[rows]), Bt, None, len(rows), K, N))
    a64 = acc.astype(np.int64)
    assert np.array_equal(a64.sum(1), A.astype(np.int64) @ Bt.astype(np.int64).sum(0))
    assert np.array_equal(a64.sum(0), Bt.astype(np.int64) @ A.astype(np.int64).sum(0))
    # gemm_int8 requant: power-of-two sc (exact-reciprocal epilogue) and a
    # generic sc; exact .5 ties (acc / 2, acc / 2 via 1/sc), overflow, and
    # sc = 0 / sa = inf (inf and NaN quantize to INT32_MIN); sc = 1 with a
    # provably small range (no range test) and with one that overflows.
    for sa, sb, sc in ((0.013, 0.7, 0.25), (1.5, -3.0, -4.0), (2.0 ** 20, 2.0 ** 20, 2.0 ** -100), (0.013, 0.7, 0.3),
                       (0.5, 1.0, 1.0), (1.0, 1.0, 2.0), (1.0, 1.0, 3.0), (0.013, 0.7, 0.0), (np.inf, 1.0, 1.0),
                       (0.013, 0.7, 1.0), (2.0 ** 20, 2.0 ** 20, 1.0)):
        out = empty((M, N), np.int32)
        say("big-tile gemm_int8", M, N, K, sa, sb, sc)
        rpl_amd.check(lib.rplhip_gemm_int8(dA.ptr, dB.ptr, out.ptr, M, N, K, sa, sb, sc, 0, 0, None))
        got = down(out, np.int32, (M, N))
        assert bits_equal(got, _requant_f32(acc, sa, sb, sc))
        ref = orc.gemm_int8(np.ascontiguousarray(A[rows]), B, len(rows), N, K, sa, sb, sc)
        assert bits_equal(got[rows], ref)
    # Zero point on A's side only (zb): acc - zb * rowsum(A), generic requant.
    zb = -7
    out = empty((M, N), np.int32)
    say("big-tile gemm_int8 zb", M, N, K)
    rpl_amd.check(lib.rplhip_gemm_int8(dA.ptr, dB.ptr, out.ptr, M, N, K, 0.013, 0.7, 0.25, 0, zb, None))
    got = down(out, np.int32, (M, N))
    rs = A.astype(np.int64).sum(1)
    acc_zb = (acc.astype(np.int64) - zb * rs[:, None]).astype(np.int32)
    assert bits_equal(got, _requant_f32(acc_zb, 0.013, 0.7, 0.25))
    assert bits_equal(got[rows], orc.gemm_int8(np.ascontiguousarray(A[rows]), B, len(rows), N, K, 0.013, 0.7, 0.25,
                                               0, zb))
    # Zero points on both sides: acc - zb * rowsum(A) - za * colsum(B) + K * za * zb
    # (the column term comes from B's column sums, taken with the transposed copy).
    za = 5
    out = empty((M, N), np.int32)
    say("big-tile gemm_int8 za zb", M, N, K)
    rpl_amd.check(lib.rplhip_gemm_int8(dA.ptr, dB.ptr, out.ptr, M, N, K, 0.013, 0.7, 0.25, za, zb, None))
    got = down(out, np.int32, (M, N))
    cs = B.astype(np.int64).sum(0)
    v = acc.astype(np.int64) - zb * rs[:, None] - za * cs[None, :] + K * za * zb
    acc_zz = ((v + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)
    assert bits_equal(got, _requant_f32(acc_zz, 0.013, 0.7, 0.25))
    assert bits_equal(got[rows], orc.gemm_int8(np.ascontiguousarray(A[rows]), B, len(rows), N, K, 0.013, 0.7, 0.25,
                                               za, zb))
    # gemm_int8_dequant: per-tensor A scale, per-column B scale, B [K,N].
    sa1 = np.float32([0.02])
    sbc = (rng.random(N).astype(np.float32) + 0.5) * np.float32(0.03)
    dsa1, dsbc, Yd = up(sa1), up(sbc), empty((M, N), np.float32)
    say("big-tile gemm_int8_dequant", M, N, K)
    rpl_amd.check(lib.rplhip_gemm_int8_dequant(dA.ptr, dsa1.ptr, 0, dB.ptr, dsbc.ptr, 1, Yd.ptr, M, N, K, None))
    assert bits_equal(down(Yd, np.float32, (M, N)), (acc.astype(np.float32) * sa1[0]) * sbc[None, :])
    # linear_int8_dequant: per-row x scales, per-column w scales, fp32 out.
    sx = (rng.random(M).astype(np.float32) + 0.5) * np.float32(0.01)
    sw = (rng.random(N).astype(np.float32) + 0.5) * np.float32(0.02)
    dsx, dsw, Y = up(sx), up(sw), empty((M, N), np.float32)
    say("big-tile linear_int8_dequant", M, N, K)
    rpl_amd.check(lib.rplhip_linear_int8_dequant(dA.ptr, dsx.ptr, 1, dBt.ptr, dsw.ptr, 1, Y.ptr, M, K, N, None))
    y = down(Y, np.float32, (M, N))
    assert bits_equal(y, (acc.astype(np.float32) * sx[:, None]) * sw[None, :])
    assert bits_equal(y[rows], orc.dequant_acc(acc[rows], sx[rows], True, sw, True))


# Skinny GEMMs (M <= 16) on the LDS-staged MFMA kernel (k_skinny_dma): full K
# slices with 4 waves (K = 8192) and 8 waves (K = 16384), partial slices
# (K = 4096 + 64, 12288), ragged N; bit-exact against the oracle, int32 and
# fused dequant.
@pytest.mark.parametrize("M,K,N", [(5, 8192, 1000), (16, 8192, 77), (8, 16384, 300), (16, 12288, 129),
                                   (12, 4160, 513), (16, 64, 40)])
def test_skinny_mfma_vs_oracle(gpu, orc, M, K, N):
    rng = np.random.default_rng(M * 31 + K + N)
    x = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    b = rng.integers(-128, 128, N, dtype=np.int8)
    say("skinny linear_int8", M, K, N)
    ref = orc.linear_int8(x, w, None, M, K, N)
    assert bits_equal(linear_int8(x, w, None, M, K, N), ref)
    assert bits_equal(linear_int8(x, w, b, M, K, N), orc.linear_int8(x, w, b, M, K, N))
    sx = (rng.random(M).astype(np.float32) + 0.5) * np.float32(0.01)
    sw = (rng.random(N).astype(np.float32) + 0.5) * np.float32(0.02)
    say("skinny linear_int8_dequant", M, K, N)
    got = linear_int8_dequant(x, sx, True, w, sw, True, M, K, N)
    assert bits_equal(got, orc.dequant_acc(ref, sx, True, sw, True))
