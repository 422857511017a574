"""rplhip_gemm_int8_noalloc (the allocation-free variant of rplhip_gemm_int8,
scratch in a static 16 MiB device array) against rplhip_gemm_int8 through the
C ABI: int32 outputs bit for bit, two calls in a row on the shared scratch
with the second one smaller, and the oracle on sampled rows.  Shapes cover the
scratch's uses: B transposed into it (N % 16 != 0, or a zero point of B),
A's row sums (zb), B's column sums (za), and B read in place (no B copy)."""
import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal
from gpu_util import down, empty, say, up

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _pair(lib, A, B, M, N, K, sa, sb, sc, za, zb):
    """Outputs of the existing entry point and of the no-alloc one."""
    dA, dB = up(A), up(B)
    ref, got = empty((M, N), np.int32), empty((M, N), np.int32)
    rpl_amd.check(lib.rplhip_gemm_int8(dA.ptr, dB.ptr, ref.ptr, M, N, K, sa, sb, sc, za, zb, None), "gemm_int8")
    rpl_amd.check(lib.rplhip_gemm_int8_noalloc(dA.ptr, dB.ptr, got.ptr, M, N, K, sa, sb, sc, za, zb, None),
                  "gemm_int8_noalloc")
    return down(ref, np.int32, (M, N)), down(got, np.int32, (M, N))


# Each sequence runs back to back on the same scratch, the second call
# smaller than the first, so stale bytes from the first would show.
SEQUENCES = [
    # B transposed into scratch (N % 16 != 0) with both zero points, then a
    # smaller ragged shape with other zero points.
    [(700, 1000, 1500, 0.013, 0.7, 0.25, 3, -5), (100, 60, 200, 0.02, 0.5, 1.0, -2, 7)],
    # Big-tile shapes: za forces the transposed copy (4 MiB of B), then B
    # read in place (256 tiles of 256 x 256) with only A's row sums in scratch.
    [(4096, 4096, 1024, 1.0, 1.0, 1.0, 1, 0), (4096, 4096, 512, 0.5, 0.25, 2.0, 0, 3)],
    # Nearly the largest copy that fits (K * N + 4 * N + 16 <= 16 MiB), then 1 x 1 x 1.
    [(64, 4096, 4091, 0.01, 0.02, 0.5, 5, 0), (1, 1, 1, 1.0, 1.0, 1.0, 0, 0)],
]


@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_noalloc_matches_gemm_int8(gpu, orc, seq):
    lib = gpu
    for i, (M, N, K, sa, sb, sc, za, zb) in enumerate(SEQUENCES[seq]):
        rng = np.random.default_rng(1000 * seq + i)
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        B = rng.integers(-128, 128, (K, N), dtype=np.int8)
        say("gemm_int8_noalloc", seq, i, M, N, K, sa, sb, sc, za, zb)
        ref, got = _pair(lib, A, B, M, N, K, sa, sb, sc, za, zb)
        assert bits_equal(got, ref)
        rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, min(M, 4), replace=False)]))
        want = orc.gemm_int8(np.ascontiguousarray(A[rows]), B, len(rows), N, K, sa, sb, sc, za, zb)
        assert bits_equal(got[rows], want)


def test_noalloc_rejects_oversized_scratch(gpu):
    """A call whose transposed B would not fit the static scratch is refused
    with RPLHIP_ERR_UNSUPPORTED and a message naming the sizes; the output
    is left untouched.  Without the zero point the same shape reads B in
    place (256 x 256 tiles, K % 64 == 0) and needs no copy."""
    lib = gpu
    M, N, K = 3072, 4096, 4160  # za != 0: B is copied, 4160 * 4096 bytes > 16 MiB
    A = np.ones((M, K), np.int8)
    B = np.ones((K, N), np.int8)
    dA, dB = up(A), up(B)
    C0 = np.full((M, N), 7, np.int32)
    dC = up(C0)
    say("gemm_int8_noalloc oversized")
    st = lib.rplhip_gemm_int8_noalloc(dA.ptr, dB.ptr, dC.ptr, M, N, K, 1.0, 1.0, 1.0, 1, 0, None)
    assert st == rpl_amd.ERR_UNSUPPORTED
    assert b"static scratch" in lib.rplhip_last_error()
    assert bits_equal(down(dC, np.int32, (M, N)), C0)
    say("gemm_int8_noalloc in place, large B")
    ref, got = _pair(lib, A, B, M, N, K, 1.0, 1.0, 1.0, 0, 0)
    assert bits_equal(got, ref)
    assert np.all(got == K)
