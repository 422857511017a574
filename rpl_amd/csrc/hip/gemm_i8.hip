// INT8 GEMMs on gfx950 i8 MFMA (v_mfma_i32_16x16x64_i8), int32 accumulation.
//
// Core kernel: NT layout (A [M,K] and B [N,K], both k-contiguous), which is
// what the MFMA operands want: every lane feeds 16 consecutive k bytes of one
// row.  Block tile BM x BN x BK staged through LDS (double-buffered, rows
// padded by 16 bytes so the 16 lanes of a ds_read_b128 phase hit distinct
// banks), 4 waves each owning a (BM/2) x (BN/2) sub-tile of 16x16 MFMA
// blocks.  Global loads are 128-bit and coalesced along k.
//
// The epilogue is fused and selected at compile time:
//   kRaw     : out = acc + bias[n]                      (linear_int8)
//   kRequant : out = x86((int32)roundf(((float)acc*sa)*sb/sc)), optional
//              zero-point correction                     (gemm_int8)
//   kDequant : y = ((float)acc * sx[m|0]) * sw[n|0]      (fused fp32 output)
//
// gemm_int8's B is [K,N] (n-contiguous); it is first transposed into a
// stream-ordered workspace so the NT core serves both layouts.
//
// M <= 16 (decode-style skinny GEMMs) runs a separate bandwidth kernel: one
// block per 16 rows of B, waves split K, each lane streams 16-byte chunks of
// B straight from HBM into MFMA operands, partial tiles reduced through LDS.
#include <math.h>

#include "common.h"

namespace {

enum Epi { kRaw = 0, kRequant = 1, kDequant = 2 };

struct EpiParams {
    // kRaw
    const int8_t* bias;  // may be NULL
    int32_t* out_i32;
    // kRequant
    float sa, sb, sc;
    int32_t za, zb;
    const int32_t* rowsum_a;  // [M], NULL when zb == 0
    const int32_t* rowsum_b;  // [N], NULL when za == 0
    int32_t kzz;              // K*za*zb (wrapping)
    // kDequant
    const float* sx;
    const float* sw;
    int sx_per_row, sw_per_col;
    float* out_f32;
    uint32_t ldc;
};

template <int EPI>
__device__ __forceinline__ void epilogue_store(const EpiParams& p, uint32_t m, uint32_t n, int32_t acc) {
    uint64_t o = (uint64_t)m * p.ldc + n;
    if (EPI == kRaw) {
        int32_t v = acc;
        if (p.bias) v = wrap_add(v, (int32_t)p.bias[n]);
        p.out_i32[o] = v;
    } else if (EPI == kRequant) {
        int32_t v = acc;
        if (p.rowsum_a) v = wrap_add(v, -wrap_mul(p.zb, p.rowsum_a[m]));
        if (p.rowsum_b) v = wrap_add(v, -wrap_mul(p.za, p.rowsum_b[n]));
        v = wrap_add(v, p.kzz);
        float result = (float)v * p.sa * p.sb / p.sc;  // ops_extended.c:119
        p.out_i32[o] = x86_cvt_i32(roundf(result));
    } else {
        float v = (float)acc * p.sx[p.sx_per_row ? m : 0];
        p.out_f32[o] = v * p.sw[p.sw_per_col ? n : 0];
    }
}

// ------------------------------------------------------------ NT core GEMM

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kPitch = BK + 16;  // bytes per LDS row
constexpr int kWaves = 4, kThreads = 64 * kWaves;
constexpr int TM = BM / 2, TN = BN / 2;  // wave tile
constexpr int FM = TM / 16, FN = TN / 16;
constexpr int kChunksA = BM * BK / 16 / kThreads;  // 16-byte chunks per thread
constexpr int kChunksB = BN * BK / 16 / kThreads;

// Load one 16-byte chunk (row r, byte column kc) of a k-contiguous tile with
// zero fill outside [rows, K).  ALIGNED: K, ld multiple of 16, base 16-aligned.
template <bool ALIGNED>
__device__ __forceinline__ v4i load_chunk(const int8_t* __restrict__ base, uint32_t ld, uint32_t rows,
                                          uint32_t K, uint32_t r, uint32_t k) {
    v4i z = {0, 0, 0, 0};
    if (r >= rows) return z;
    const int8_t* p = base + (uint64_t)r * ld + k;
    if (ALIGNED) {
        if (k >= K) return z;
        return *reinterpret_cast<const v4i*>(p);
    } else {
        union {
            v4i v;
            int8_t b[16];
        } u;
#pragma unroll
        for (int i = 0; i < 16; i++) u.b[i] = (k + i < K) ? p[i] : (int8_t)0;
        return u.v;
    }
}

template <int EPI, bool ALIGNED>
__global__ void __launch_bounds__(kThreads) k_gemm_i8_nt(const int8_t* __restrict__ A, uint32_t lda,
                                                         const int8_t* __restrict__ B, uint32_t ldb,
                                                         uint32_t M, uint32_t N, uint32_t K, EpiParams p) {
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * kPitch];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * kPitch];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64, wave = tid / 64;
    const uint32_t wm = wave / 2, wn = wave % 2;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v4i){0, 0, 0, 0};

    v4i ra[kChunksA], rb[kChunksB];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < kChunksA; i++) {
            uint32_t c = tid + i * kThreads;
            uint32_t r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            ra[i] = load_chunk<ALIGNED>(A, lda, M, K, m0 + r, k0 + kc);
        }
#pragma unroll
        for (int i = 0; i < kChunksB; i++) {
            uint32_t c = tid + i * kThreads;
            uint32_t r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            rb[i] = load_chunk<ALIGNED>(B, ldb, N, K, n0 + r, k0 + kc);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kChunksA; i++) {
            uint32_t c = tid + i * kThreads;
            uint32_t r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            *reinterpret_cast<v4i*>(&As[buf][r * kPitch + kc]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kChunksB; i++) {
            uint32_t c = tid + i * kThreads;
            uint32_t r = c / (BK / 16), kc = (c % (BK / 16)) * 16;
            *reinterpret_cast<v4i*>(&Bs[buf][r * kPitch + kc]) = rb[i];
        }
    };

    const uint32_t nk = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK / 64; kk++) {
            v4i a[FM], b[FN];
            const uint32_t kofs = kk * 64 + (lane / 16) * 16;
#pragma unroll
            for (int i = 0; i < FM; i++)
                a[i] = *reinterpret_cast<const v4i*>(&As[buf][(wm * TM + i * 16 + lane % 16) * kPitch + kofs]);
#pragma unroll
            for (int j = 0; j < FN; j++)
                b[j] = *reinterpret_cast<const v4i*>(&Bs[buf][(wn * TN + j * 16 + lane % 16) * kPitch + kofs]);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // D layout of a 16x16 MFMA block: lane holds column lane%16, rows
    // 4*(lane/16) + r in element r.
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                uint32_t m = m0 + wm * TM + i * 16 + 4 * (lane / 16) + r;
                uint32_t n = n0 + wn * TN + j * 16 + lane % 16;
                if (m < M && n < N) epilogue_store<EPI>(p, m, n, acc[i][j][r]);
            }
}

// --------------------------------------------------- skinny (M <= 16) GEMM

constexpr int kSkWaves = 8, kSkThreads = 64 * kSkWaves, kSkUnroll = 8;

template <int EPI, bool ALIGNED>
__global__ void __launch_bounds__(kSkThreads) k_gemv_i8_nt(const int8_t* __restrict__ A, uint32_t lda,
                                                           const int8_t* __restrict__ B, uint32_t ldb,
                                                           uint32_t M, uint32_t N, uint32_t K,
                                                           uint32_t k_per_wave, EpiParams p) {
    __shared__ v4i red[kSkWaves][64];
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t n0 = blockIdx.x * 16;
    const uint32_t ra = lane % 16, rb = n0 + lane % 16;
    const uint32_t kl = (lane / 16) * 16;
    const uint32_t kbeg = wave * k_per_wave;
    const uint32_t kend = kbeg + k_per_wave < K ? kbeg + k_per_wave : K;

    v4i acc = {0, 0, 0, 0};
    for (uint32_t k = kbeg; k < kend; k += 64 * kSkUnroll) {
        v4i a[kSkUnroll], b[kSkUnroll];
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++) {
            uint32_t kk = k + u * 64 + kl;
            bool in = k + u * 64 < kend;
            b[u] = in ? load_chunk<ALIGNED>(B, ldb, N, K, rb, kk) : (v4i){0, 0, 0, 0};
            a[u] = in ? load_chunk<ALIGNED>(A, lda, M, K, ra, kk) : (v4i){0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < kSkWaves; w++) {
        v4i t = red[w][lane];
        acc[0] = wrap_add(acc[0], t[0]);
        acc[1] = wrap_add(acc[1], t[1]);
        acc[2] = wrap_add(acc[2], t[2]);
        acc[3] = wrap_add(acc[3], t[3]);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        uint32_t m = 4 * (lane / 16) + r, n = n0 + lane % 16;
        if (m < M && n < N) epilogue_store<EPI>(p, m, n, acc[r]);
    }
}

// ----------------------------------------------------- helpers for gemm_int8

// Bt[n][k] = B[k][n] through a 64x64 LDS tile.
__global__ void __launch_bounds__(256) k_transpose_i8(const int8_t* __restrict__ B, uint32_t K, uint32_t N,
                                                      int8_t* __restrict__ Bt) {
    __shared__ int8_t t[64][65];
    const uint32_t k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    for (uint32_t i = threadIdx.x; i < 64 * 64; i += 256) {
        uint32_t r = i / 64, c = i % 64;
        uint32_t k = k0 + r, n = n0 + c;
        t[r][c] = (k < K && n < N) ? B[(uint64_t)k * N + n] : (int8_t)0;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < 64 * 64; i += 256) {
        uint32_t r = i / 64, c = i % 64;  // r: n offset, c: k offset
        uint32_t n = n0 + r, k = k0 + c;
        if (n < N && k < K) Bt[(uint64_t)n * K + k] = t[c][r];
    }
}

// rowsum[r] = sum_k X[r][k] (int32) for the zero-point correction.
__global__ void __launch_bounds__(256) k_rowsum_i8(const int8_t* __restrict__ X, uint32_t rows, uint32_t K,
                                                   int32_t* __restrict__ out) {
    __shared__ int32_t s[4];
    uint32_t r = blockIdx.x;
    int32_t acc = 0;
    for (uint32_t k = threadIdx.x; k < K; k += 256) acc += X[(uint64_t)r * K + k];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (threadIdx.x % 64 == 0) s[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[r] = s[0] + s[1] + s[2] + s[3];
}

// --------------------------------------------------------------- dispatch

bool aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

template <int EPI>
int run_nt(const int8_t* A, uint32_t lda, const int8_t* B, uint32_t ldb, uint32_t M, uint32_t N, uint32_t K,
           const EpiParams& p, hipStream_t s) {
    bool al = K % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && aligned16(A) && aligned16(B);
    if (M <= 16) {
        // Split K over the block's waves in 64-byte steps.
        uint32_t kpw = (K + kSkWaves - 1) / kSkWaves;
        kpw = (kpw + 63) / 64 * 64;
        dim3 grid((N + 15) / 16);
        if (al)
            hipLaunchKernelGGL((k_gemv_i8_nt<EPI, true>), grid, dim3(kSkThreads), 0, s, A, lda, B, ldb, M, N, K,
                               kpw, p);
        else
            hipLaunchKernelGGL((k_gemv_i8_nt<EPI, false>), grid, dim3(kSkThreads), 0, s, A, lda, B, ldb, M, N, K,
                               kpw, p);
        return rplhip::check_launch("skinny int8 GEMM");
    }
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    if (grid.y > 65535) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "int8 GEMM: M=%u too large", M);
    if (al)
        hipLaunchKernelGGL((k_gemm_i8_nt<EPI, true>), grid, dim3(kThreads), 0, s, A, lda, B, ldb, M, N, K, p);
    else
        hipLaunchKernelGGL((k_gemm_i8_nt<EPI, false>), grid, dim3(kThreads), 0, s, A, lda, B, ldb, M, N, K, p);
    return rplhip::check_launch("int8 GEMM");
}

int transpose_b(const int8_t* B, uint32_t K, uint32_t N, int8_t* Bt, hipStream_t s) {
    dim3 grid((N + 63) / 64, (K + 63) / 64);
    if (grid.y > 65535) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "int8 transpose: K=%u too large", K);
    hipLaunchKernelGGL(k_transpose_i8, grid, dim3(256), 0, s, B, K, N, Bt);
    return rplhip::check_launch("int8 transpose");
}

}  // namespace

using namespace rplhip;

extern "C" {

int rplhip_linear_int8(const int8_t* X, const int8_t* W, const int8_t* bias, int32_t* out, uint32_t M,
                       uint32_t K, uint32_t N, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!out || (K && (!X || !W))) return fail(RPLHIP_ERR_INVALID, "rplhip_linear_int8: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    EpiParams p = {};
    p.bias = bias;
    p.out_i32 = out;
    p.ldc = N;
    return run_nt<kRaw>(X, K, W, K, M, N, K, p, as_stream(stream));
}

int rplhip_linear_int8_dequant(const int8_t* X, const float* x_scale, int x_per_row, const int8_t* W,
                               const float* w_scale, int w_per_row, float* Y, uint32_t M, uint32_t K,
                               uint32_t N, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!Y || !x_scale || !w_scale || (K && (!X || !W)))
        return fail(RPLHIP_ERR_INVALID, "rplhip_linear_int8_dequant: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    EpiParams p = {};
    p.sx = x_scale;
    p.sw = w_scale;
    p.sx_per_row = x_per_row;
    p.sw_per_col = w_per_row;
    p.out_f32 = Y;
    p.ldc = N;
    return run_nt<kDequant>(X, K, W, K, M, N, K, p, as_stream(stream));
}

int rplhip_gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K,
                     float sa, float sb, float sc, int32_t za, int32_t zb, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!C || (K && (!A || !B))) return fail(RPLHIP_ERR_INVALID, "rplhip_gemm_int8: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    size_t bt_bytes = ((size_t)K * N + 15) / 16 * 16;
    size_t sums = (za ? (size_t)N : 0) + (zb ? (size_t)M : 0);
    void* ws = nullptr;
    int st = ws_alloc(&ws, bt_bytes + sizeof(int32_t) * sums + 16, s);
    if (st) return st;
    int8_t* Bt = (int8_t*)ws;
    int32_t* sum_ptr = (int32_t*)((char*)ws + bt_bytes);
    EpiParams p = {};
    p.out_i32 = C;
    p.ldc = N;
    p.sa = sa;
    p.sb = sb;
    p.sc = sc;
    p.za = za;
    p.zb = zb;
    p.kzz = (int32_t)((uint32_t)K * (uint32_t)za * (uint32_t)zb);
    if (K) st = transpose_b(B, K, N, Bt, s);
    if (!st && zb && K) {
        p.rowsum_a = sum_ptr;
        sum_ptr += M;
        hipLaunchKernelGGL(k_rowsum_i8, dim3(M), dim3(256), 0, s, A, M, K, (int32_t*)p.rowsum_a);
        st = check_launch("int8 row sums");
    }
    if (!st && za && K) {
        p.rowsum_b = sum_ptr;
        hipLaunchKernelGGL(k_rowsum_i8, dim3(N), dim3(256), 0, s, Bt, N, K, (int32_t*)p.rowsum_b);
        st = check_launch("int8 column sums");
    }
    if (!st) st = run_nt<kRequant>(A, K, Bt, K, M, N, K, p, s);
    ws_free(ws, s);
    return st;
}

int rplhip_gemm_int8_dequant(const int8_t* A, const float* a_scale, int a_per_row, const int8_t* B,
                             const float* b_scale, int b_per_col, float* Y, uint32_t M, uint32_t N, uint32_t K,
                             rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!Y || !a_scale || !b_scale || (K && (!A || !B)))
        return fail(RPLHIP_ERR_INVALID, "rplhip_gemm_int8_dequant: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    void* ws = nullptr;
    int st = ws_alloc(&ws, ((size_t)K * N + 15) / 16 * 16 + 16, s);
    if (st) return st;
    EpiParams p = {};
    p.sx = a_scale;
    p.sw = b_scale;
    p.sx_per_row = a_per_row;
    p.sw_per_col = b_per_col;
    p.out_f32 = Y;
    p.ldc = N;
    if (K) st = transpose_b(B, K, N, (int8_t*)ws, s);
    if (!st) st = run_nt<kDequant>(A, K, (const int8_t*)ws, K, M, N, K, p, s);
    ws_free(ws, s);
    return st;
}

}  // extern "C"
