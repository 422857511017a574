"""Helpers for the GPU parity tests: device buffers through the C ABI."""
import ctypes as C
import sys

import numpy as np

import rpl_amd
from rpl_amd import DeviceBuffer, check


def say(*a):
    """Name the case before each GPU step (flushed, so a fault still shows it)."""
    print(*a, flush=True)
    sys.stdout.flush()


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, dtype, shape):
    check(rpl_amd.lib().rplhip_synchronize(), "sync")
    return buf.to_array(dtype, shape)


def empty(shape, dtype):
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return DeviceBuffer(max(n, 1))


def sgemm(A, B, C0, M, N, K, alpha=1.0, beta=0.0, ta=False, tb=False, lda=None, ldb=None, ldc=None):
    lib = rpl_amd.lib()
    dA, dB, dC = up(A), up(B), up(C0)
    lda = lda or (M if ta else K)
    ldb = ldb or (K if tb else N)
    ldc = ldc or N
    check(lib.rplhip_sgemm(int(ta), int(tb), M, N, K, alpha, dA.ptr, lda, dB.ptr, ldb, beta, dC.ptr, ldc, None),
          "sgemm")
    return down(dC, np.float32, C0.shape)


def gemm_int8(A, B, M, N, K, sa=1.0, sb=1.0, sc=1.0, za=0, zb=0):
    lib = rpl_amd.lib()
    dA, dB, dC = up(A), up(B), empty((M, N), np.int32)
    check(lib.rplhip_gemm_int8(dA.ptr, dB.ptr, dC.ptr, M, N, K, sa, sb, sc, za, zb, None), "gemm_int8")
    return down(dC, np.int32, (M, N))


def linear_int8(x, w, bias, M, K, N):
    lib = rpl_amd.lib()
    dx, dw, do = up(x), up(w), empty((M, N), np.int32)
    db = up(bias) if bias is not None else None
    check(lib.rplhip_linear_int8(dx.ptr, dw.ptr, db.ptr if db else None, do.ptr, M, K, N, None), "linear_int8")
    return down(do, np.int32, (M, N))


def linear_int8_dequant(x, sx, x_per_row, w, sw, w_per_row, M, K, N):
    lib = rpl_amd.lib()
    dx, dw, dsx, dsw = up(x), up(w), up(np.float32(sx).reshape(-1)), up(np.float32(sw).reshape(-1))
    dy = empty((M, N), np.float32)
    check(lib.rplhip_linear_int8_dequant(dx.ptr, dsx.ptr, int(x_per_row), dw.ptr, dsw.ptr, int(w_per_row), dy.ptr,
                                         M, K, N, None), "linear_int8_dequant")
    return down(dy, np.float32, (M, N))


def gemm_err_ratio(C, A, B, C_ref, alpha=1.0, beta=0.0, C0=None):
    """max |C - C_ref| / (|alpha| sum_k |a b| + |beta||C0|), in float64."""
    denom = abs(alpha) * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))
    if C0 is not None and beta:
        denom = denom + abs(beta) * np.abs(C0.astype(np.float64))
    denom = np.maximum(denom, 1e-300)
    return float(np.max(np.abs(C.astype(np.float64) - C_ref.astype(np.float64)) / denom))


def fp32_tol(K):
    """The fp32 GEMM parity bound: max rel err <= 1e-5 * sqrt(K)."""
    return 1e-5 * np.sqrt(max(K, 1))


def np_ptr(a, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))
