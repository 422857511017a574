// INT8 GEMMs on gfx950, int32 accumulation.
//
// All kernels take the NT layout (A [M,K] and B [N,K], both k-contiguous),
// which is what the i8 MFMA operands want: every lane feeds 16 consecutive
// k-bytes of one row.  gemm_int8's B is [K,N] (n-contiguous); it is first
// transposed into a workspace so the NT kernels serve both layouts.
//
// Which kernel runs (run_nt):
//   M <= 16, K % 64 == 0, K <= 16384, aligned : k_skinny, an HBM-streaming
//       kernel (whole rows of B per load instruction, VGPR landing, LDS
//       permute into v_mfma_i32_16x16x64_i8 fragments, waves split K).
//   M <= 4 otherwise                          : k_gemv_i8_dot4 (VALU dot4).
//   4 < M <= 16 otherwise                     : k_gemv_i8_nt (MFMA, byte-safe).
//   >= 2 tiles of 256 x 256 per CU, aligned, K % 64 == 0, operands < 2 GiB :
//       k_gemm_i8_nt_dma, 256 x 256 x 64 tiles, one wave per SIMD with a
//       128 x 128 wave tile of v_mfma_i32_32x32x32_i8 (accumulators in
//       AGPRs), HBM -> LDS copies done by the load unit (buffer_load ... lds)
//       into a 4-stage ring, epilogue stored straight from the accumulators.
//   everything else                           : k_gemm_i8_nt<Cfg<128,128>>
//       (or <256,256> for big unaligned-K shapes), register-staged pipeline,
//       byte-safe loads for odd K / alignment.
// Tiles are visited in an XCD-aware grouped order (rplhip::tile_of): the 8
// XCDs each take a contiguous range of tiles, walked 8 tile-rows at a time,
// so the A and B panels an XCD's 32 CUs share stay in that XCD's L2.
//
// The epilogue is fused and selected at compile time:
//   kRaw         : out = acc + bias[n]                       (linear_int8)
//   kRequant     : out = x86((int32)roundf(((float)acc*sa)*sb/sc)), optional
//                  zero-point correction                      (gemm_int8)
//   kRequantPow2 : kRequant with sc = +-2^k, where x/sc == x*(1/sc) exactly
//   kRequantUnit : kRequant with sc = 1 and |acc*sa*sb| < 2^30 proven on the
//                  host (no NaN, no overflow): no divide and no range test
//   kDequant     : y = ((float)acc * sx[m|0]) * sw[n|0]       (fused fp32 output)
#include <math.h>
#include <pthread.h>
#include <stdlib.h>

#include <type_traits>

#include "mfma_pipe.h"

namespace {

using rplhip::lds_ptr;
using rplhip::static_for;
using rplhip::swz;
using rplhip::tile_of;
using rplhip::uniform_rsrc;
using rplhip::waitcnt_imm;

enum Epi { kRaw = 0, kRequant = 1, kDequant = 2, kRequantPow2 = 3, kRequantUnit = 4 };

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
    // kRequantPow2 (no zero points, sc = +-2^k with 1/sc exact): x / sc is
    // computed as x * inv_sc, which rounds the same real number once.
    float inv_sc;
    // kDequant
    const float* sx;
    const float* sw;
    int sx_per_row, sw_per_col;
    float* out_f32;
    uint32_t ldc;
};

// The column and row terms of the epilogue, loaded once per column / row by
// the tile epilogues: cadd (kRaw: bias[n]; kRequant: -za * rowsum_b[n]),
// cmul (kDequant: sw[n]), radd (kRequant: -zb * rowsum_a[m]) and rmul
// (kDequant: sx[m]); 0 where the variant has none.  The int32 products and
// negations wrap, as the reference's x86 arithmetic does.
template <int EPI>
__device__ __forceinline__ int32_t epi_cadd(const EpiParams& p, uint32_t n) {
    if constexpr (EPI == kRaw) return p.bias ? (int32_t)p.bias[n] : 0;
    if constexpr (EPI == kRequant) return p.rowsum_b ? (int32_t)(0u - (uint32_t)wrap_mul(p.za, p.rowsum_b[n])) : 0;
    return 0;
}
template <int EPI>
__device__ __forceinline__ float epi_cmul(const EpiParams& p, uint32_t n) {
    if constexpr (EPI == kDequant) return p.sw[p.sw_per_col ? n : 0];
    return 0.0f;
}
template <int EPI>
__device__ __forceinline__ int32_t epi_radd(const EpiParams& p, uint32_t m) {
    if constexpr (EPI == kRequant) return p.rowsum_a ? (int32_t)(0u - (uint32_t)wrap_mul(p.zb, p.rowsum_a[m])) : 0;
    return 0;
}
template <int EPI>
__device__ __forceinline__ float epi_rmul(const EpiParams& p, uint32_t m) {
    if constexpr (EPI == kDequant) return p.sx[p.sx_per_row ? m : 0];
    return 0.0f;
}

// Output bits of one element from its accumulator and the terms of its
// column (cadd, cmul) and row (radd, rmul); the int32 sums wrap, so their
// order does not matter, and the float operation order is the reference's
// (src/ops_extended.c:119).
template <int EPI>
__device__ __forceinline__ uint32_t epi_bits(const EpiParams& p, int32_t acc, int32_t cadd, float cmul, int32_t radd,
                                             float rmul) {
#pragma clang fp contract(off)
    if constexpr (EPI == kRaw) {
        return (uint32_t)wrap_add(acc, cadd);
    } else if constexpr (EPI == kRequant) {
        int32_t v = wrap_add(wrap_add(acc, radd), cadd);
        v = wrap_add(v, p.kzz);
        return (uint32_t)x86_round_cvt((float)v * p.sa * p.sb / p.sc);
    } else if constexpr (EPI == kRequantPow2) {
        return (uint32_t)x86_round_cvt((float)acc * p.sa * p.sb * p.inv_sc);
    } else if constexpr (EPI == kRequantUnit) {
        // x86_round_cvt without its range test (the sum is within +-2^30).
        const float y = (float)acc * p.sa * p.sb;
        return (uint32_t)(int32_t)(y + __builtin_copysignf(0.49999997f, y));
    } else {
        return __float_as_uint((float)acc * rmul * cmul);
    }
}

template <int EPI>
__device__ __forceinline__ void epilogue_store(const EpiParams& p, uint32_t m, uint32_t n, int32_t acc) {
    const uint64_t o = (uint64_t)m * p.ldc + n;
    const uint32_t bits = epi_bits<EPI>(p, acc, epi_cadd<EPI>(p, n), epi_cmul<EPI>(p, n), epi_radd<EPI>(p, m),
                                        epi_rmul<EPI>(p, m));
    if constexpr (EPI == kDequant)
        p.out_f32[o] = __uint_as_float(bits);
    else
        p.out_i32[o] = (int32_t)bits;
}

// Load one 16-byte chunk (row r, byte column k) of a k-contiguous matrix with
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

// As load_chunk, for data read exactly once (weights of the decode GEMVs):
// the aligned path uses a non-temporal load, which streams a 64 MiB matrix
// from HBM ~8% faster than a plain load (measured on MI355X).
template <bool ALIGNED>
__device__ __forceinline__ v4i load_chunk_stream(const int8_t* __restrict__ base, uint32_t ld, uint32_t rows,
                                                 uint32_t K, uint32_t r, uint32_t k) {
    if (ALIGNED && r < rows && k < K)
        return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(base + (uint64_t)r * ld + k));
    return load_chunk<ALIGNED>(base, ld, rows, K, r, k);
}

// ------------------------------------------------------------ NT core GEMM

// MFMA: v_mfma_i32_32x32x32_i8 (65536 ops, 32 cycles).  It sustains ~95% of
// the i8 peak from one wave per SIMD, where 16x16x64 with the same number of
// accumulator registers stalls near 60% (measured on MI355X).  Operand
// layout: lane l feeds row (or column) l%32 of the 32x32 block with the 16
// k-bytes 16*(l/32) .. +16 of the 32-k step; the int32 result element r of
// lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
//
// Pipeline: three LDS stages, two fragment register sets and two register
// sets of in-flight HBM loads.  In iteration kt the MFMAs consume tile kt
// from registers, while the same wave reads tile kt+1's fragments out of
// LDS, writes tile kt+2 (fetched two iterations earlier) into LDS, and
// issues the HBM loads of tile kt+4; one barrier per iteration.  LDS latency
// is hidden behind 32 MFMAs and HBM/L2 latency behind two iterations.  The
// steady-state iterations carry no conditions (edge tiles and the last
// iterations run a separate, checked copy of the loop), which lets the
// compiler wait only for the loads it needs (vmcnt) instead of draining.
// LDS rows are unpadded 64-byte k-slices with XOR-swizzled 16-byte chunks
// (rplhip::swz).

template <int BM_, int BN_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = 64;
    static constexpr int kThreads = 256;            // 4 waves, 2 x 2
    static constexpr int TM = BM / 2, TN = BN / 2;  // wave tile
    static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave tile
    static constexpr int kPitch = BK;  // LDS row pitch in bytes (swizzled, unpadded)
    static constexpr int kChunksA = BM * BK / 16 / kThreads;
    static constexpr int kChunksB = BN * BK / 16 / kThreads;
    static constexpr int kCPR = BK / 16;  // 16-byte chunks per tile row
    static constexpr int kStages = 4;
    static constexpr int kStageBytes = (BM + BN) * kPitch;
    // Epilogue staging: one 32 x TN int32 block-row per wave, padded so
    // that rows 4 apart (the two lane halves of a store) use disjoint banks.
    static constexpr int kEpiPitch = TN + 8;
    static_assert(4 * 32 * kEpiPitch * 4 <= kStages * kStageBytes, "epilogue staging must fit the LDS stages");
};

using CfgBig = Cfg<256, 256>;
using CfgSmall = Cfg<128, 128>;

// Fragments of one 32-k step.
template <class G>
struct Frags {
    v4i a[G::FM], b[G::FN];
};

// Fused epilogue of rows m0..m0+3 of column n (a lane's 4 results of a
// 16 x 16 MFMA block), with the terms loaded before the first store (stores
// count in vmcnt: a load between them would wait for every earlier one).
template <int EPI>
__device__ __forceinline__ void epilogue_store_rows4(const EpiParams& p, uint32_t m0, uint32_t n, uint32_t M,
                                                     uint32_t N, v4i v) {
    if (n >= N) return;
    const int32_t cadd = epi_cadd<EPI>(p, n);
    const float cmul = epi_cmul<EPI>(p, n);
    int32_t radd[4];
    float rmul[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {  // rows past M read row M-1, never stored
        radd[r] = epi_radd<EPI>(p, m0 + r < M ? m0 + r : M - 1);
        rmul[r] = epi_rmul<EPI>(p, m0 + r < M ? m0 + r : M - 1);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));  // the stores below need no vmcnt wait
#pragma unroll
    for (int r = 0; r < 4; r++) {
        if (m0 + r >= M) break;
        const uint64_t o = (uint64_t)(m0 + r) * p.ldc + n;
        const uint32_t bits = epi_bits<EPI>(p, v[r], cadd, cmul, radd[r], rmul[r]);
        if constexpr (EPI == kDequant)
            p.out_f32[o] = __uint_as_float(bits);
        else
            p.out_i32[o] = (int32_t)bits;
    }
}

// Fused epilogue on 4 consecutive columns n..n+3 of row m, given the
// columns' and the row's terms.
template <int EPI>
__device__ __forceinline__ void epilogue_store4(const EpiParams& p, uint32_t m, uint32_t n, uint32_t N, v4i v,
                                                const int32_t (&cadd)[4], const float (&cmul)[4], int32_t radd,
                                                float rmul) {
    const uint64_t o = (uint64_t)m * p.ldc + n;
    void* out = EPI == kDequant ? (void*)(p.out_f32 + o) : (void*)(p.out_i32 + o);
    v4i r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = (int32_t)epi_bits<EPI>(p, v[e], cadd[e], cmul[e], radd, rmul);
    if (n + 3 < N && (p.ldc & 3) == 0 && (((uintptr_t)out) & 15) == 0) {
        *reinterpret_cast<v4i*>(out) = r;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (n + e < N) reinterpret_cast<int32_t*>(out)[e] = r[e];
    }
}

template <class G, int EPI, bool ALIGNED>
__global__ void __launch_bounds__(256, 1) k_gemm_i8_nt(const int8_t* __restrict__ A, uint32_t lda,
                                                       const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                       uint32_t N, uint32_t K, EpiParams p) {
    constexpr int BM = G::BM, BN = G::BN, BK = G::BK, TM = G::TM, TN = G::TN, FM = G::FM, FN = G::FN;
    constexpr int P = G::kPitch, CPR = G::kCPR, S = G::kStages;
    __shared__ __attribute__((aligned(16))) int8_t smem[S * G::kStageBytes];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % 64, wave = tid / 64;
    const uint32_t wm = wave / 2, wn = wave % 2;
    uint32_t im, in;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, im, in);
    const uint32_t m0 = im * BM, n0 = in * BN;

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v16i){};

    struct Ld {
        v4i a[G::kChunksA], b[G::kChunksB];
    };
    // HBM -> registers for one k-tile.  The fast path uses raw buffer loads:
    // one resource per operand based at the tile's first row and sized to
    // the rows that exist, so rows past M / N read as zeros in hardware; the
    // lane's byte offset is one VGPR and the chunk / k offsets are scalars.
    // It needs K % 64 == 0 and operands under 2 GiB; anything else takes
    // the guarded element path.
    const uint32_t voff_a = (tid / CPR) * lda + (tid % CPR) * 16;
    const uint32_t voff_b = (tid / CPR) * ldb + (tid % CPR) * 16;
    constexpr uint32_t kRowsPerLoad = G::kThreads / CPR;
    const __amdgpu_buffer_rsrc_t rsrc_a = uniform_rsrc(A + (uint64_t)m0 * lda, (M > m0 ? M - m0 : 0) * lda);
    const __amdgpu_buffer_rsrc_t rsrc_b = uniform_rsrc(B + (uint64_t)n0 * ldb, (N > n0 ? N - n0 : 0) * ldb);
    auto gload_fast = [&](uint32_t k0, Ld& g) {
#pragma unroll
        for (int i = 0; i < G::kChunksA; i++)
            g.a[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a, k0 + i * kRowsPerLoad * lda, 0);
#pragma unroll
        for (int i = 0; i < G::kChunksB; i++)
            g.b[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b, k0 + i * kRowsPerLoad * ldb, 0);
    };
    auto gload_edge = [&](uint32_t k0, Ld& g) {
#pragma unroll
        for (int i = 0; i < G::kChunksA; i++) {
            uint32_t c = tid + i * G::kThreads;
            g.a[i] = load_chunk<ALIGNED>(A, lda, M, K, m0 + c / CPR, k0 + (c % CPR) * 16);
        }
#pragma unroll
        for (int i = 0; i < G::kChunksB; i++) {
            uint32_t c = tid + i * G::kThreads;
            g.b[i] = load_chunk<ALIGNED>(B, ldb, N, K, n0 + c / CPR, k0 + (c % CPR) * 16);
        }
    };
    auto sstore = [&](uint32_t stage, const Ld& g) {
        int8_t* As = smem + stage * G::kStageBytes;
        int8_t* Bs = As + BM * P;
#pragma unroll
        for (int i = 0; i < G::kChunksA; i++) {
            uint32_t c = tid + i * G::kThreads, r = c / CPR;
            *reinterpret_cast<v4i*>(&As[r * P + ((c % CPR) ^ swz(r)) * 16]) = g.a[i];
        }
#pragma unroll
        for (int i = 0; i < G::kChunksB; i++) {
            uint32_t c = tid + i * G::kThreads, r = c / CPR;
            *reinterpret_cast<v4i*>(&Bs[r * P + ((c % CPR) ^ swz(r)) * 16]) = g.b[i];
        }
    };
    // MFMA operand fragments of 32-k step kk of the tile in `stage`: lane
    // feeds row lane%32 of each 32-row block with 16-byte chunk
    // 2*kk + lane/32.
    auto fload = [&](uint32_t stage, int kk, Frags<G>& f) {
        const int8_t* As = smem + stage * G::kStageBytes;
        const int8_t* Bs = As + BM * P;
        const uint32_t ch = 2 * kk + lane / 32;
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const uint32_t r = wm * TM + i * 32 + lane % 32;
            f.a[i] = *reinterpret_cast<const v4i*>(&As[r * P + (ch ^ swz(r)) * 16]);
        }
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const uint32_t r = wn * TN + j * 32 + lane % 32;
            f.b[j] = *reinterpret_cast<const v4i*>(&Bs[r * P + (ch ^ swz(r)) * 16]);
        }
    };
    auto mma = [&](const Frags<G>& f) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    };

    const uint32_t nk = (K + BK - 1) / BK;
    auto mainloop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto gload = [&](uint32_t k0, Ld& g) {
            if constexpr (FAST) gload_fast(k0, g);
            else gload_edge(k0, g);
        };
        // Prologue: tiles 0 and 1 into LDS stages 0 and 1, tiles 2 and 3
        // in flight in the two load sets.
        Ld g0, g1;
        gload(0, g0);
        sstore(0, g0);
        if (nk > 1) {
            gload(BK, g1);
            sstore(1, g1);
        }
        if (nk > 2) gload(2 * BK, g0);
        if (nk > 3) gload(3 * BK, g1);
        __syncthreads();
        Frags<G> f0, f1;
        fload(0, 0, f0);
        // Iteration kt (f0 holds tile kt's first 32-k step on entry, the
        // load set in use holds tile kt+2): store tile kt+2 to LDS, fetch
        // tile kt+4, then alternate fragment reads and MFMAs one 32-k step
        // ahead, ending with f0 holding tile kt+1's first step.  The barrier
        // protects the stage that a later iteration overwrites.
        //
        // Steady state unrolled by the stage count, so every stage index is
        // a compile-time constant (LDS addresses fold into immediates); the
        // two load sets alternate at compile time.
        uint32_t kt = 0;
        for (; kt + S + 3 < nk; kt += S) {
            static_for<S>([&](auto U) {
                constexpr int u = decltype(U)::value;
                Ld& g = (u & 1) ? g1 : g0;
                sstore((u + 2) % S, g);
                gload((kt + u + 4) * BK, g);
                fload(u, 1, f1);
                mma(f0);
                fload((u + 1) % S, 0, f0);
                mma(f1);
                __syncthreads();
            });
        }
        // Last iterations: identical code each time (the load sets rotate by
        // value), so the accumulators' dataflow never forks -- a fork makes
        // the register allocator give them a second home.  On entry g0
        // holds tile kt+2 and g1 tile kt+3.
        for (; kt < nk; kt++) {
            if (kt + 2 < nk) sstore((kt + 2) % S, g0);
            g0 = g1;
            if (kt + 4 < nk) gload((kt + 4) * BK, g1);
            fload(kt % S, 1, f1);
            mma(f0);
            if (kt + 1 < nk) fload((kt + 1) % S, 0, f0);
            mma(f1);
            __syncthreads();
        }
    };
    if (ALIGNED && K % BK == 0 && (uint64_t)M * lda < (1ull << 31) && (uint64_t)N * ldb < (1ull << 31))
        mainloop(std::true_type{});
    else
        mainloop(std::false_type{});

    // Epilogue through LDS: each wave stages one 32-row block-row of its
    // tile, then reads it back row-major so every lane owns 4 consecutive
    // columns and stores them with one 128-bit write.  The block-row index
    // is a compile-time constant (static_for), so the accumulators are never
    // indexed dynamically (which would force them out of registers).
    int32_t* stage = reinterpret_cast<int32_t*>(smem) + wave * 32 * G::kEpiPitch;
    constexpr int kLanesPerRow = TN / 4;
    constexpr int kRowsPerPass = 64 / kLanesPerRow, kPasses = 32 / kRowsPerPass;
    const uint32_t row0 = lane / kLanesPerRow, col = (lane % kLanesPerRow) * 4, n = n0 + wn * TN + col;
    // The column and row terms of every element the lane stores, all
    // loaded and waited for before the first store (stores count in vmcnt:
    // a load between them, or a wait the compiler cannot count through the
    // stores' branches, would wait for every earlier store).  Columns and
    // rows past N and M read the last one, never stored.
    int32_t cadd[4], radd[FM][kPasses];
    float cmul[4], rmul[FM][kPasses];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        cadd[e] = epi_cadd<EPI>(p, n + e < N ? n + e : N - 1);
        cmul[e] = epi_cmul<EPI>(p, n + e < N ? n + e : N - 1);
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int k = 0; k < kPasses; k++) {
            const uint32_t m = m0 + wm * TM + i * 32 + k * kRowsPerPass + row0;
            radd[i][k] = epi_radd<EPI>(p, m < M ? m : M - 1);
            rmul[i][k] = epi_rmul<EPI>(p, m < M ? m : M - 1);
        }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    static_for<FM>([&](auto I) {
        constexpr int i = decltype(I)::value;
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                stage[(8 * (r / 4) + 4 * (lane / 32) + r % 4) * G::kEpiPitch + j * 32 + lane % 32] = acc[i][j][r];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kPasses; k++) {
            const uint32_t row = k * kRowsPerPass + row0;
            const v4i v = *reinterpret_cast<const v4i*>(&stage[row * G::kEpiPitch + col]);
            const uint32_t m = m0 + wm * TM + i * 32 + row;
            if (m < M && n < N) epilogue_store4<EPI>(p, m, n, N, v, cadd, cmul, radd[i][k], rmul[i][k]);
        }
        __syncthreads();
    });
}

// Fused epilogue straight from MFMA accumulators: FM x FN blocks of 32x32
// (acc may be wider, FNA >= FN columns, the rest unused);
// result register r of lane l in block (i, j) is row mb + i*32 + 8*(r/4) +
// r%4 and column nb + j*32, where mb = tile row + 4*(l/32) and nb = tile
// column + l%32.  Fully unrolled (the accumulators are only ever indexed by
// constants); values that depend on the column are loaded once per block
// column, those that depend on the row once per row.  Each store
// instruction writes two 128-byte row segments.  This is the bounds-checked
// form for edge tiles; epilogue_tile_full serves interior ones.
template <int EPI, int FM, int FN, int FNA = FN>
__device__ __forceinline__ void epilogue_tile(const EpiParams& p, const v16i (&acc)[FM][FNA], uint32_t mb,
                                              uint32_t nb, uint32_t M, uint32_t N) {
    // The column and row terms of all the lane's elements, loaded and
    // waited for before the first store (stores count in vmcnt: a load
    // between them, or a wait the compiler cannot count through the stores'
    // bounds branches, would wait for every earlier store).  Columns and
    // rows past N and M read the last one, never stored.
    int32_t cadd[FN];
    float cmul[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const uint32_t n = nb + j * 32;
        cadd[j] = epi_cadd<EPI>(p, n < N ? n : N - 1);
        cmul[j] = epi_cmul<EPI>(p, n < N ? n : N - 1);
    }
    int32_t radd[FM][16];
    float rmul[FM][16];
    static_for<FM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<16>([&](auto R) {
            constexpr int r = decltype(R)::value;
            const uint32_t m = mb + i * 32 + 8 * (r / 4) + r % 4;
            radd[i][r] = epi_radd<EPI>(p, m < M ? m : M - 1);
            rmul[i][r] = epi_rmul<EPI>(p, m < M ? m : M - 1);
        });
    });
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    static_for<FM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<16>([&](auto R) {
            constexpr int r = decltype(R)::value;
            const uint32_t m = mb + i * 32 + 8 * (r / 4) + r % 4;
            if (m >= M) return;
            static_for<FN>([&](auto J) {
                constexpr int j = decltype(J)::value;
                const uint32_t n = nb + j * 32;
                if (n < N) {
                    const uint32_t bits = epi_bits<EPI>(p, acc[i][j][r], cadd[j], cmul[j], radd[i][r], rmul[i][r]);
                    const uint64_t o = (uint64_t)m * p.ldc + n;
                    if constexpr (EPI == kDequant)
                        p.out_f32[o] = __uint_as_float(bits);
                    else
                        p.out_i32[o] = (int32_t)bits;
                }
            });
        });
    });
}

// Cache policy of the full-tile epilogue's stores: 2 = non-temporal (the
// output is written once and not read back by the GEMM).  Measured at
// 8192^3 (gemm_int8): 0.4405 ms against 0.4476 with the default policy.
#ifndef RPL_I8_EPI_CPOL
#define RPL_I8_EPI_CPOL 2
#endif

// Largest ldc for which a 128-row wave sub-tile spans < 2^31 bytes of C.
constexpr uint32_t kFullEpiMaxLdc = 1u << 21;

// The same for a wave sub-tile of FM*32 x FN*32 outputs that lies wholly
// inside C (origin wm0, wn0, wave-uniform), with FM*32*ldc*4 < 2^31.  The
// stores are raw buffer stores whose address needs no VALU work: the
// resource is based at the sub-tile origin, the lane's part (row 4*(l/32),
// column l%32) is one VGPR offset, the row of result register r (a
// constant times ldc) goes in the scalar offset and the 32-column block in
// the instruction's immediate offset.
template <int EPI, int FM, int FN, int FNA = FN>
__device__ __forceinline__ void epilogue_tile_full(const EpiParams& p, const v16i (&acc)[FM][FNA], uint32_t wm0,
                                                   uint32_t wn0, uint32_t lane) {
    const uint32_t ldc4 = p.ldc * 4;
    const void* out = EPI == kDequant ? (const void*)p.out_f32 : (const void*)p.out_i32;
    const __amdgpu_buffer_rsrc_t rsrc =
        uniform_rsrc((const char*)out + ((uint64_t)wm0 * p.ldc + wn0) * 4, FM * 32 * ldc4);
    const uint32_t voff = 4 * (lane / 32) * ldc4 + (lane % 32) * 4;
    const uint32_t mb = wm0 + 4 * (lane / 32), nb = wn0 + lane % 32;
    int32_t cadd[FN];
    float cmul[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        cadd[j] = epi_cadd<EPI>(p, nb + j * 32);
        cmul[j] = epi_cmul<EPI>(p, nb + j * 32);
    }
    // The row terms of all the lane's rows before the first store (stores
    // count in vmcnt: a load between them would wait for every earlier one).
    int32_t radd[FM][16];
    float rmul[FM][16];
    static_for<FM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<16>([&](auto R) {
            constexpr int r = decltype(R)::value;
            radd[i][r] = epi_radd<EPI>(p, mb + i * 32 + 8 * (r / 4) + r % 4);
            rmul[i][r] = epi_rmul<EPI>(p, mb + i * 32 + 8 * (r / 4) + r % 4);
        });
    });
    static_for<FM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<16>([&](auto R) {
            constexpr int r = decltype(R)::value;
            constexpr uint32_t row = i * 32 + 8 * (r / 4) + r % 4;
            const int soff = (int)__builtin_amdgcn_readfirstlane(row * ldc4);
            static_for<FN>([&](auto J) {
                constexpr int j = decltype(J)::value;
                const uint32_t bits = epi_bits<EPI>(p, acc[i][j][r], cadd[j], cmul[j], radd[i][r], rmul[i][r]);
                __builtin_amdgcn_raw_buffer_store_b32(bits, rsrc, (int)(voff + j * 128), soff, RPL_I8_EPI_CPOL);
            });
        });
    });
}

// ------------------------------------ NT core GEMM, direct-to-LDS pipeline


// Tuning knob (default measured best on MI355X): LDS stages in the ring.
// (6 stages for the 256 x 128 tile, which fit, measured the same as 4.)
#ifndef RPL_I8_STAGES
#define RPL_I8_STAGES 4
#endif

namespace dma {
constexpr int BM = 256, BK = 64, S = RPL_I8_STAGES, kThreads = 256;
// [K][N] B tiles: k-row r keeps its logical 16-byte chunk c in physical
// chunk c ^ kn_swz(r % 8).  Measured on gfx950 (SQ_LDS_BANK_CONFLICT per
// ds_read_b64_tr_b8 of the fragment pattern): moving chunk bits 1-3 reads
// without conflicts; any XOR that moves chunk bit 0 (the two 16-lane groups
// reading adjacent chunks) costs 2 extra cycles per read.
__device__ __forceinline__ uint32_t kn_swz(uint32_t e) { return 2 * e; }
typedef __attribute__((address_space(3))) v2i* lds_v2i;
// ds_read_b64_tr_b8 through a restrict parameter: inlining gives the read
// alias-scope metadata, as the kernel's plain LDS reads have.  Without it
// the compiler's wait insertion cannot tell the read from the in-flight
// direct-to-LDS copies and waits for all of them (vmcnt(0)) before every
// first read of a half, which serialises the copy pipeline.  The copies a
// read depends on are waited for explicitly (vmcnt + barrier), as for the
// A fragments.
__device__ __forceinline__ v2i tr8(lds_v2i __restrict__ p) { return __builtin_amdgcn_ds_read_tr8_b64_v2i32(p); }
// B-tile height BN = 256 (the big tile) or 128 (grids with too few 256 x
// 256 tiles to fill the chip): 4 waves (2 x 2), wave tile 128 x BN/2.
template <int BN>
struct Geo {
    static_assert(BN == 256 || BN == 128, "B tile of 256 or 128 rows");
    static constexpr int kStages = S;
    static_assert(kStages >= 3 && kStages * (BM + BN) * BK <= 160 * 1024, "LDS ring must fit 160 KB");
    static constexpr int FN = BN / 64;                    // 32-wide MFMA blocks per wave (N side)
    static constexpr int kTileBytesA = BM * BK;           // A part of one stage: 16 KB
    static constexpr int kStageBytes = (BM + BN) * BK;
    static constexpr int kLoadsA = BM / 64, kLoadsB = BN / 64;  // 1 KB copies per wave per tile
    static constexpr int kVmPerTile = kLoadsA + kLoadsB;  // copy instructions per wave per tile
};
// Fragments of one 32-k half: 4 A blocks and either FN B blocks (B [N,K])
// or the two 8-byte transposed halves of each B block (BKN).
template <bool BKN, int FN>
struct HalfFrags;
template <int FN>
struct HalfFrags<false, FN> {
    v4i a[4], b[FN];
    __device__ v4i bv(int j) const { return b[j]; }
};
template <int FN>
struct HalfFrags<true, FN> {
    v4i a[4];
    v2i bl[FN], bh[FN];
    __device__ v4i bv(int j) const { return (v4i){bl[j].x, bl[j].y, bh[j].x, bh[j].y}; }
};
// Fragment reads of a half, in the order its MFMAs (A block m / FN, B block
// m % FN) first use them: A block 0, the B reads, A blocks 1..3.  Read r < 4
// is A block r; then B block r - 4 (B [N,K]) or the low / high half of B
// block (r - 4) / 2 (BKN).
template <bool BKN, int FN>
__device__ constexpr int read_at(int m) {
    constexpr int nb = (BKN ? 2 : 1) * FN;
    return m == 0 ? 0 : m <= nb ? 3 + m : m - nb;
}
}  // namespace dma

// Same tiles, MFMA and fused epilogues as k_gemm_i8_nt<CfgBig>, with the
// HBM -> LDS copies done by the load unit itself (buffer_load_dwordx4 ...
// lds): each instruction moves 16 rows x 64 bytes of a tile into 1 KB of
// LDS, lane l writing bytes 16l..16l+15.  The XOR swizzle of the LDS rows is
// produced by choosing which 16-byte chunk each lane fetches (lane l of a
// load fetches chunk (l%4) ^ swz(row) of row l/4), so the fragment reads
// stay conflict-free and no VGPRs or ds_write instructions stage the tiles.
//
// Pipeline over a ring of 4 LDS stages: tile kt+3 is requested while tile kt
// is multiplied; one barrier per tile, placed between the two 32-k halves,
// after which the wave's own copies of tile kt+1 have landed (explicit
// vmcnt) and every wave has finished reading the stage that the next
// iteration refills.  Rows past M / N are clamped to the last row (their
// products are never stored), so no load leaves the operand.
//
// The epilogue stores straight from the accumulators: for each of the 16
// result registers a wave writes two 128-byte row segments (32 lanes x 4
// bytes each), so every store fills whole cache lines.
//
// Requires K % 64 == 0, 16-byte aligned operands and leading dimensions,
// and operands below 2 GiB (32-bit buffer offsets).
//
// BKN: B is stored [K][N] (row k at B + k*ldb, the layout of gemm_int8's
// B) and is read in place, with no transposed copy.  A B stage is then 64
// k-rows of 256 bytes: each copy instruction moves 4 k-rows, lane l writing
// 16-byte chunk l%16 of row l/16, fetched from logical chunk
// (l%16) ^ 2*(k%8).  The fragments come from ds_read_b64_tr_b8: within each
// 16-lane group, lane 2e+h addresses 8 bytes (columns 8h..8h+7 of the
// group's 16-column chunk) of k-row k0+e, and output lane 8h+b receives
// byte b of lane 2e+h's piece as its byte e, i.e. column 8h+b at k-rows
// k0..k0+7.  Two such reads give a lane the 16 k-bytes of its column that
// the MFMA's B operand holds, in the same k order as the A fragment.  The
// eight k-rows of one read sit in 8 distinct 16-byte chunks of their rows
// (dma::kn_swz).  Needs BN = 256, N % 16 == 0.
template <int EPI, int BN, bool BKN = false>
__global__ void __launch_bounds__(256, 1) k_gemm_i8_nt_dma(const int8_t* __restrict__ A, uint32_t lda,
                                                           const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                           uint32_t N, uint32_t K, EpiParams p) {
    using dma::BK;
    using dma::BM;
    using G = dma::Geo<BN>;
    constexpr int S = G::kStages;
    constexpr int FN = G::FN, kLoadsA = G::kLoadsA, kLoadsB = G::kLoadsB, kVmPerTile = G::kVmPerTile;
    constexpr int kTileBytesA = G::kTileBytesA, kStageBytes = G::kStageBytes;
    static_assert(!BKN || BN == 256, "[K][N] B needs 256-column tiles");
    __shared__ __attribute__((aligned(1024))) int8_t smem[S * kStageBytes];

    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t wm = wave / 2, wn = wave % 2;
    uint32_t im, in;
    tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, im, in);
    const uint32_t m0 = im * BM, n0 = in * BN;
    const uint32_t rows_a = M - m0 < (uint32_t)BM ? M - m0 : BM;
    const uint32_t rows_b = N - n0 < (uint32_t)BN ? N - n0 : BN;
    const __amdgpu_buffer_rsrc_t rsrc_a = uniform_rsrc(A + (uint64_t)m0 * lda, rows_a * lda);
    // [K][N] B: the resource starts at column n0 and ends after column N-1
    // of row K-1.
    const __amdgpu_buffer_rsrc_t rsrc_b = BKN ? uniform_rsrc(B + n0, (K - 1) * ldb + rows_b)
                                              : uniform_rsrc(B + (uint64_t)n0 * ldb, rows_b * ldb);

    // Source offsets of this lane's A and B copies (k added as the scalar
    // offset): wave w copies rows w*BM/4 .. and w*BN/4 .. of the tiles.
    // (Array bounds here must not depend on BN: the host pass of hipcc then
    // drops the kernel's launch stub without a diagnostic.  Sized for the
    // largest tile; loops run to kLoadsA / kLoadsB / FN.)
    uint32_t voff_a[4], voff_b[4];
#pragma unroll
    for (int i = 0; i < kLoadsA; i++) {
        const uint32_t r = wave * (BM / 4) + i * 16 + lane / 4;
        voff_a[i] = (r < rows_a ? r : rows_a - 1) * lda + ((lane % 4) ^ swz(r)) * 16;
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; i++) {
        if constexpr (BKN) {
            // k-row r of the tile; chunks past the last column (N % 256 != 0)
            // are clamped to the last one, so every load stays inside B.
            // Copies i and i+2 are 8 k-rows apart with the same chunks: the
            // 8 rows go in the scalar offset, so only i = 0, 1 take VGPRs.
            if (i >= 2) continue;
            const uint32_t r = wave * 16 + i * 4 + lane / 16;
            const uint32_t c = (lane % 16) ^ dma::kn_swz(r % 8);
            voff_b[i] = r * ldb + (16 * c < rows_b ? c : rows_b / 16 - 1) * 16;
        } else {
            const uint32_t r = wave * (BN / 4) + i * 16 + lane / 4;
            voff_b[i] = (r < rows_b ? r : rows_b - 1) * ldb + ((lane % 4) ^ swz(r)) * 16;
        }
    }
    auto issue_a = [&](uint32_t kt, uint32_t stage) {
        int8_t* st = smem + stage * kStageBytes;
#pragma unroll
        for (int i = 0; i < kLoadsA; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_ptr)(st + (wave * (BM / 4) + i * 16) * BK), 16,
                                                     voff_a[i], kt * BK, 0, 0);
    };
    auto issue_b = [&](uint32_t kt, uint32_t stage) {
        int8_t* st = smem + stage * kStageBytes;
#pragma unroll
        for (int i = 0; i < kLoadsB; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc_b, (lds_ptr)(st + kTileBytesA + (wave * (BN / 4) + i * 16) * BK), 16, voff_b[BKN ? i % 2 : i],
                BKN ? (kt * BK + 8 * (i / 2)) * ldb : kt * BK, 0, 0);
    };
    auto issue = [&](uint32_t kt, uint32_t stage) {
        issue_a(kt, stage);
        issue_b(kt, stage);
    };
    // Wait until this wave's copies of tile kt+1 have landed, given that
    // `later` whole tiles (plus `extra` single copies) were issued after it.
    auto wait_after = [&](uint32_t later) {
        static_for<S - 1>([&](auto C) {
            constexpr int c = decltype(C)::value;
            if (later == (uint32_t)c) __builtin_amdgcn_s_waitcnt(waitcnt_imm(c * kVmPerTile, 0));
        });
    };

    // Fragment reads: lane feeds row lane%32 of each 32-row block with chunk
    // 2*kk + lane/32; the rows of a block differ from lane%32 by a multiple
    // of 32, so the swizzle slot depends on the lane alone.
    const uint32_t fr = lane % 32;
    uint32_t foff[2];
#pragma unroll
    for (int kk = 0; kk < 2; kk++) foff[kk] = fr * BK + ((2 * kk + lane / 32) ^ swz(fr)) * 16;
    const uint32_t a_base = wm * 128 * BK, b_base = kTileBytesA + wn * (BN / 2) * BK;
    // [K][N] B: lane 16g + 2e + h reads k-row 16(g/2) + e (+ 32kk + 8t) at
    // columns 128wn + 32j + 16(g%2) + 8h, in chunk (8wn + 2j + g%2) ^ kn_swz(e).
    uint32_t boff[4];
    if constexpr (BKN) {
        const uint32_t g = lane / 16, e = (lane % 16) / 2, h = lane % 2;
#pragma unroll
        for (int j = 0; j < 4; j++)
            boff[j] = kTileBytesA + (16 * (g / 2) + e) * 256 + ((8 * wn + 2 * j + g % 2) ^ dma::kn_swz(e)) * 16 + 8 * h;
    }
    using F = dma::HalfFrags<BKN, FN>;
    using dma::lds_v2i;
    constexpr int kReads = 4 + (BKN ? 2 : 1) * FN;  // fragment reads per half
    // Read r of stage `stage`, k-half kk (r as in dma::read_at).
    auto read_one = [&](uint32_t stage, int kk, int r, F& f) {
        const int8_t* st = smem + stage * kStageBytes;
        if (r < 4) {
            f.a[r] = *reinterpret_cast<const v4i*>(st + foff[kk] + a_base + r * 32 * BK);
        } else if constexpr (BKN) {
            const int j = (r - 4) / 2, hi = (r - 4) % 2;
            const v2i t = dma::tr8((lds_v2i)(st + kk * 32 * 256 + boff[j] + hi * 8 * 256));
            if (hi)
                f.bh[j] = t;
            else
                f.bl[j] = t;
        } else {
            f.b[r - 4] = *reinterpret_cast<const v4i*>(st + foff[kk] + b_base + (r - 4) * 32 * BK);
        }
    };
    auto fload = [&](uint32_t stage, int kk, F& f) {
        static_for<kReads>([&](auto R) { read_one(stage, kk, decltype(R)::value, f); });
    };
    v16i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v16i){};
    auto mma = [&](const F& f) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.bv(j), acc[i][j], 0, 0, 0);
    };
    // Copy c of tile kt's copies (A copies first, then B) into `stage`.
    auto copy_one = [&](uint32_t kt, uint32_t stage, int c) {
        int8_t* st = smem + stage * kStageBytes;
        if (c < kLoadsA) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_ptr)(st + (wave * (BM / 4) + c * 16) * BK), 16,
                                                     voff_a[c], kt * BK, 0, 0);
        } else {
            const int i = c - kLoadsA;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc_b, (lds_ptr)(st + kTileBytesA + (wave * (BN / 4) + i * 16) * BK), 16, voff_b[BKN ? i % 2 : i],
                BKN ? (kt * BK + 8 * (i / 2)) * ldb : kt * BK, 0, 0);
        }
    };
    // Copies of a tile issued in the first half of an iteration (the rest in
    // the second): with the half's fragment reads, at most one memory
    // instruction more than MFMAs in either half.
    constexpr int kCopiesFirst = (kVmPerTile + 1) / 2;
    // One half: its 4*FN MFMAs on `cur`, each followed by the next memory
    // instruction of the half -- the kReads fragment reads of `nxt`, then
    // copies c0 .. c0 + NC - 1 of tile kt_copy -- with a scheduling barrier
    // after each (left alone, the scheduler bunches the reads just before
    // their first use and the copies together, and the wave stalls in front
    // of its next MFMA).  When the half has more memory instructions than
    // MFMAs, its last MFMAs take two each.
    auto half = [&](const F& cur, F& nxt, uint32_t rstage, int kk, uint32_t kt_copy, uint32_t cstage, auto C0,
                    auto NC) {
        constexpr int c0 = decltype(C0)::value, nc = decltype(NC)::value, nm = 4 * FN;
        constexpr int ops = kReads + nc, two = ops > nm ? ops - nm : 0;
        static_for<nm>([&](auto Mc) {
            constexpr int m = decltype(Mc)::value;
            acc[m / FN][m % FN] =
                __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[m / FN], cur.bv(m % FN), acc[m / FN][m % FN], 0, 0, 0);
            constexpr int first = m < nm - two ? m : (nm - two) + 2 * (m - (nm - two));
            constexpr int count = m < nm - two ? 1 : 2;
            static_for<count>([&](auto Oc) {
                constexpr int o = first + decltype(Oc)::value;
                if constexpr (o < kReads)
                    read_one(rstage, kk, dma::read_at<BKN, FN>(o), nxt);
                else if constexpr (o < ops)
                    copy_one(kt_copy, cstage, c0 + o - kReads);
            });
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    const uint32_t nk = K / BK;
    // Prologue: tiles 0 .. S-2 requested, tile 0 landed and visible.
    static_for<S - 1>([&](auto T) {
        constexpr int t = decltype(T)::value;
        if (t < nk) issue(t, t);
    });
    wait_after(nk - 1 < (uint32_t)(S - 2) ? nk - 1 : S - 2);  // tiles 1 .. min(S-2, nk-1) may stay in flight
    __builtin_amdgcn_s_barrier();
    F f0, f1;
    fload(0, 0, f0);

    // Iteration kt: request tile kt+S-1 (into the stage tile kt-1 left, free
    // since the barrier of iteration kt-1), read tile kt's second half while
    // multiplying its first, wait for tile kt+1 and barrier, read tile kt+1's
    // first half while multiplying kt's second.
    // Copies issued after tile kt+1's at the barrier of iteration kt.
    constexpr int kLaterSteady = (S - 3) * kVmPerTile + kCopiesFirst;
    uint32_t kt = 0;
    for (; kt + 2 * S - 1 <= nk; kt += S) {
        static_for<S>([&](auto U) {
            constexpr int u = decltype(U)::value;
            const uint32_t tc = kt + u + S - 1, sc = (u + S - 1) % S;
            __builtin_amdgcn_sched_barrier(0);
            half(f0, f1, u, 1, tc, sc, std::integral_constant<int, 0>{},
                 std::integral_constant<int, kCopiesFirst>{});
            __builtin_amdgcn_s_waitcnt(waitcnt_imm(kLaterSteady, 0));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            half(f1, f0, (u + 1) % S, 0, tc, sc, std::integral_constant<int, kCopiesFirst>{},
                 std::integral_constant<int, kVmPerTile - kCopiesFirst>{});
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    // Last iterations: a whole tile is requested in the first half.
    for (; kt < nk; kt++) {
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        fload(kt % S, 1, f1);
        mma(f0);
        const uint32_t last = kt + S - 1 < nk - 1 ? kt + S - 1 : nk - 1;  // last tile requested so far
        wait_after(last > kt + 1 ? last - kt - 1 : 0);
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < nk) fload((kt + 1) % S, 0, f0);
        mma(f1);
    }

    if (m0 + BM <= M && n0 + BN <= N && p.ldc <= kFullEpiMaxLdc)
        epilogue_tile_full<EPI, 4, FN, 4>(p, acc, m0 + wm * 128, n0 + wn * (BN / 2), lane);
    else
        epilogue_tile<EPI, 4, FN, 4>(p, acc, m0 + wm * 128 + 4 * (lane / 32), n0 + wn * (BN / 2) + lane % 32, M,
                                     N);
}

// ------------------- big-tile GEMM with operands copied two k-steps at a time
//
// Same tile (256 x BN x 64, 4 waves of 128 x BN/2 on v_mfma_i32_32x32x32_i8)
// and fused epilogues as k_gemm_i8_nt_dma<EPI, BN, BKN>, with A, and B
// [N,K], copied in k-step pairs: one copy instruction moves 8 rows x 128
// bytes (8 whole cache lines; the per-k-step copy moves 16 rows x 64 bytes,
// half of 16 lines, and fetches each line twice; whole lines copy 1.5-1.75x
// faster than half lines under the same access pattern, measured on
// MI355X).  A pair of A tiles
// fills a 32 KB region laid out in 1 KB row groups: group g holds rows
// 8g..8g+7, the first 512 bytes k-step 2p, the next 512 bytes k-step 2p+1,
// each as 8 rows x 64 bytes with chunk c at slot c ^ swz(row).  Lane l of a
// copy writes bytes 16l..16l+15 of one group, so it fetches k-step l/32, row
// 8g + (l%32)/4, chunk (l%4) ^ swz(row).  (Keying the swizzle on row % 8
// alone leaves rows 8 apart on the same banks: measured 4 extra cycles per
// read.)  Fragment reads then see the per-k-step layout (64-byte rows, the
// same swizzle) at a parity offset of 0 or 512 bytes.  B [N,K] pairs use the
// same layout over BN rows.  B [K,N] (BKN) keeps the per-k-step stages of
// k_gemm_i8_nt_dma (its rows are whole 256-byte segments already).  LDS: two
// A pair slots (64 KB; three, 96 KB, at BN = 128, whose LDS has the room),
// then four B stages (BKN, 64 KB) or three B pair slots (96 KB at BN = 256,
// 48 KB at 128).
//
// Instruction schedule.  Each 32-k half issues its 4 FN MFMAs with one other
// memory instruction after each (two after the last ones when there are
// more): the 12 (BKN) or 4 + FN fragment reads of the next half, then
// kLoadsB = BN/64 B copies (first half) or 4 A copies (second half).  Copies
// issued in clusters stall the wave in front of its next MFMA: with the
// copies bunched, a 64-k step took 1262 cycles against 1024 of MFMA work,
// spread out 1082 (s_memtime stamps per wave on MI355X, 8192^3).  Iteration
// j (tile j):
//   first half:  MFMAs on k-half 0, reads of k-half 1, and B copies: BKN, B
//                tile j+3 into stage (j+3)%4 (tile j-1's, free since the
//                barrier of iteration j-1); B [N,K], copies 0..kLoadsB-1
//                (j even) or the rest (j odd) of B pair q = j/2 + 2 into slot
//                q%3 (pair q-3's, free since the barrier of iteration 2q-5);
//   wait for tile j+1 (vmcnt(kLoadsB) when j is odd, vmcnt(2 kLoadsB + 4)
//                when even), barrier;
//   second half: MFMAs on k-half 1, reads of tile j+1's k-half 0, and half
//                an A pair: j odd, copies 0..3 of pair (j+3)/2 into tile j's
//                pair slot (free since this barrier); j even, copies 4..7 of
//                pair (j+2)/2.  With three A slots the pairs are (j+5)/2 and
//                (j+4)/2, into the slot of pair (j-1)/2 (free since this
//                barrier).
// A B [N,K] pair is complete two iterations before its first read, and the
// copy count between two waits is the one of the per-k-step B ring, so with
// two A slots the waits are the same for both B layouts.  With three, the B
// copies bind: vmcnt(2 kLoadsB + 8) when j is odd, vmcnt(3 kLoadsB + 12)
// when even.  Every iteration issues the same
// copies: copies of tiles past the end re-load the last tile (or pair) into
// a stage or slot that no later read uses, so the wait counts hold to the
// end and every access stays inside the operands.  Requires K % 128 == 0 and
// the conditions of k_gemm_i8_nt_dma.

namespace dma {
constexpr int kPairBytes = BM * 2 * BK;  // 256 rows x 128 k-bytes
}  // namespace dma

template <int EPI, bool BKN, int BN>
__device__ __forceinline__ void gemm_i8_pairs_tile(const int8_t* __restrict__ A, uint32_t lda,
                                                   const int8_t* __restrict__ B, uint32_t ldb, uint32_t M, uint32_t N,
                                                   uint32_t K, const EpiParams& p) {
    using dma::BK;
    using dma::BM;
    using dma::kPairBytes;
    static_assert(BN == 256 || (BN == 128 && !BKN), "B tiles of 256 rows, or 128 rows of B [N,K]");
    constexpr int S = 4, FN = BN / 64, kLoadsB = BN / 64;
    // A pair slots: three for 256 x 128 tiles, whose LDS has room (their A
    // copies then start two k-steps earlier), two for 256 x 256.  B [K,N]:
    // a ring of S k-step stages.  B [N,K]: three k-step pair slots laid out
    // as A's (BN rows instead of 256).
    constexpr int kASlots = BN == 128 ? 3 : 2;
    constexpr int kBStage = BN * BK, kBPairBytes = BN * 2 * BK, kBBase = kASlots * kPairBytes;
    constexpr int kBBytes = BKN ? S * kBStage : 3 * kBPairBytes;
    static_assert(kBBase + kBBytes <= 160 * 1024, "LDS must fit 160 KB");
    constexpr int kReads = BKN ? 12 : 4 + FN;  // fragment reads per half
    __shared__ __attribute__((aligned(1024))) int8_t smem[kBBase + kBBytes];

    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t wm = wave / 2, wn = wave % 2;
    const uint32_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN, nkt = K / BK;
    const uint32_t fr = lane % 32;
    uint32_t foff_a[2], foff_b[2], boff[4];
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
        foff_a[kk] = wm * 16 * 1024 + (fr / 8) * 1024 + (fr % 8) * BK + ((2 * kk + lane / 32) ^ swz(fr)) * 16;
        foff_b[kk] = (BKN ? wn * (BN / 2) * BK + fr * BK : wn * (BN / 16) * 1024 + (fr / 8) * 1024 + (fr % 8) * BK) +
                     ((2 * kk + lane / 32) ^ swz(fr)) * 16;
    }
    if constexpr (BKN) {
        const uint32_t g = lane / 16, e = (lane % 16) / 2, h = lane % 2;
#pragma unroll
        for (int j = 0; j < 4; j++)
            boff[j] = (16 * (g / 2) + e) * 256 + ((8 * wn + 2 * j + g % 2) ^ dma::kn_swz(e)) * 16 + 8 * h;
    }
    using F = dma::HalfFrags<BKN, FN>;
    using dma::lds_v2i;
    v16i acc[4][4];

    // k-steps [k0, k0 + nks) (even, >= 2) of the tile at (m0, n0), added
    // into acc.  Leaves no copy in flight and every wave past a barrier.
    auto mainloop = [&](uint32_t m0, uint32_t n0, uint32_t k0, uint32_t nks) {
        const uint32_t rows_a = M - m0 < (uint32_t)BM ? M - m0 : BM;
        const uint32_t rows_b = N - n0 < (uint32_t)BN ? N - n0 : BN;
        const __amdgpu_buffer_rsrc_t rsrc_a = uniform_rsrc(A + (uint64_t)m0 * lda, rows_a * lda);
        const __amdgpu_buffer_rsrc_t rsrc_b = BKN ? uniform_rsrc(B + n0, (K - 1) * ldb + rows_b)
                                                  : uniform_rsrc(B + (uint64_t)n0 * ldb, rows_b * ldb);
        // A pair copies: wave w fills row groups 8w .. 8w+7 (rows 64w ..
        // 64w+63); copy i covers rows R = 64w + 8i + a_rr.  The chunk swizzle
        // is swz(R), with R % 32 = 8(i%4) + a_rr, so swz(R) = swz(a_rr) ^
        // 2(i%2): the column offset of copy i is a_col ^ 32(i%2).  Rows past M
        // are clamped to the last row (never stored).
        const uint32_t a_rr = (lane % 32) / 4;
        const uint32_t a_row = wave * 64 + a_rr;
        const uint32_t a_col = (lane / 32) * BK + ((lane % 4) ^ swz(a_rr)) * 16;
        auto copy_a = [&](uint32_t pair, uint32_t aofs, int i) {  // aofs: the slot's byte offset
            int8_t* st = smem + aofs + wave * 8 * 1024;
            const uint32_t r = a_row + 8 * i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_ptr)(st + i * 1024), 16,
                                                     (r < rows_a ? r : rows_a - 1) * lda + (a_col ^ (32 * (i % 2))),
                                                     (k0 + 2 * pair) * BK, 0, 0);
        };
        // BKN: B copies as in k_gemm_i8_nt_dma, k-step kt into stage `bofs`
        // (byte offset in the B region).  B [N,K]: copy i of pair `pair` into
        // the pair slot at `bofs`, laid out as A's: wave w fills row groups
        // (BN/32)w .. (BN/32)w + BN/32 - 1, copy i rows R = (BN/4)w + 8i +
        // a_rr (BN/4 is a multiple of 16, so swz(R) = swz(a_rr) ^ 2(i%2) as
        // for A).
        uint32_t voff_b[2];
        if constexpr (BKN) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t r = wave * 16 + i * 4 + lane / 16;
                const uint32_t c = (lane % 16) ^ dma::kn_swz(r % 8);
                voff_b[i] = r * ldb + (16 * c < rows_b ? c : rows_b / 16 - 1) * 16;
            }
        }
        auto copy_b = [&](uint32_t kt, uint32_t bofs, int i) {
            int8_t* st = smem + kBBase + bofs;
            if constexpr (BKN) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_ptr)(st + (wave * (BN / 4) + i * 16) * BK), 16,
                                                         voff_b[i % 2], ((k0 + kt) * BK + 8 * (i / 2)) * ldb, 0, 0);
            } else {
                const uint32_t r = wave * (BN / 4) + 8 * i + a_rr;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rsrc_b, (lds_ptr)(st + (wave * (BN / 32) + i) * 1024), 16,
                    (r < rows_b ? r : rows_b - 1) * ldb + (a_col ^ (32 * (i % 2))), (k0 + 2 * kt) * BK, 0, 0);
            }
        };
        // Read r of k-half kk of the k-step at parity par of the A pair slot
        // at byte offset aofs and at byte offset `bofs` in the B region (BKN:
        // its stage; B [N,K]: its pair slot plus 512 par): r < 4 is A block
        // r; then B block (r-4) (B [N,K]) or the low / high transposed half
        // of B block (r-4)/2 (BKN).
        auto read_one = [&](uint32_t aofs, uint32_t par, uint32_t bofs, int kk, int r, F& f) {
            if (r < 4) {
                const int8_t* sa_ = smem + aofs + par * 512 + foff_a[kk];
                f.a[r] = *reinterpret_cast<const v4i*>(sa_ + r * 4096);
            } else if constexpr (BKN) {
                const int j = (r - 4) / 2, hi = (r - 4) % 2;
                const int8_t* pb = smem + kBBase + bofs + kk * 32 * 256 + boff[j] + hi * 8 * 256;
                const v2i t = dma::tr8((lds_v2i)pb);
                if (hi)
                    f.bh[j] = t;
                else
                    f.bl[j] = t;
            } else {
                f.b[r - 4] = *reinterpret_cast<const v4i*>(smem + kBBase + bofs + foff_b[kk] + (r - 4) * 4096);
            }
        };
        // One half: its 4*FN MFMAs on `cur`, each followed by the next
        // memory instruction of the half -- read o of `nxt` (o < kReads),
        // then copy o - kReads of the half's NC -- with the last MFMAs taking
        // two when the half has more memory instructions than MFMAs (256 x
        // 128 tiles: 10 for 8).
        auto half = [&](const F& cur, F& nxt, uint32_t aofs, uint32_t par, uint32_t bofs, int kk, auto NCc,
                        auto copy) {
            constexpr int nc = decltype(NCc)::value, nm = 4 * FN, ops = kReads + nc;
            constexpr int two = ops > nm ? ops - nm : 0;
            static_for<nm>([&](auto Mc) {
                constexpr int m = decltype(Mc)::value;
                acc[m / FN][m % FN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[m / FN], cur.bv(m % FN),
                                                                           acc[m / FN][m % FN], 0, 0, 0);
                constexpr int first = m < nm - two ? m : (nm - two) + 2 * (m - (nm - two));
                constexpr int count = m < nm - two ? 1 : 2;
                static_for<count>([&](auto Oc) {
                    constexpr int o = first + decltype(Oc)::value;
                    if constexpr (o < kReads)
                        read_one(aofs, par, bofs, kk, dma::read_at<BKN, FN>(o), nxt);
                    else if constexpr (o < ops)
                        copy(o - kReads);
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        };

        // Prologue: A pair 0 (tiles 0, 1), B tiles 0..2 (BKN) or B pairs 0, 1
        // (slots 0, 1), then copies 0..3 of A pair 1 (two A slots) or all of
        // A pair 1 and copies 0..3 of A pair 2 (three); tile 0 landed.  The
        // waits before a tile's first read allow the copies issued after its
        // last one: with two A slots kLoadsB when the tile is even (the A
        // copies of the iteration before and the current B copies) and
        // 2 kLoadsB + 4 when odd; with three (B binds: its last copies are
        // two iterations back) 2 kLoadsB + 8 and 3 kLoadsB + 12.
        const uint32_t npairs = nks / 2;
        constexpr int kWaitEvenTile = kASlots == 3 ? 2 * kLoadsB + 8 : kLoadsB;
        constexpr int kWaitOddTile = kASlots == 3 ? 3 * kLoadsB + 12 : 2 * kLoadsB + 4;
#pragma unroll
        for (int i = 0; i < 8; i++) copy_a(0, 0, i);
        if constexpr (BKN) {
#pragma unroll
            for (int t = 0; t < 3; t++) {
                const uint32_t src = (uint32_t)t < nks ? t : nks - 1;
#pragma unroll
                for (int i = 0; i < kLoadsB; i++) copy_b(src, t * kBStage, i);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const uint32_t src = (uint32_t)q < npairs ? q : npairs - 1;
#pragma unroll
                for (int i = 0; i < 2 * kLoadsB; i++) copy_b(src, q * kBPairBytes, i);
            }
        }
        if constexpr (kASlots == 3) {
#pragma unroll
            for (int i = 0; i < 8; i++) copy_a(npairs > 1 ? 1 : 0, kPairBytes, i);
#pragma unroll
            for (int i = 0; i < 4; i++) copy_a(npairs > 2 ? 2 : npairs - 1, 2 * kPairBytes, i);
            __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * kLoadsB + 12, 0));
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) copy_a(npairs > 1 ? 1 : 0, kPairBytes, i);
            __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * kLoadsB + 4, 0));
        }
        __builtin_amdgcn_s_barrier();
        F f0, f1;
        static_for<kReads>([&](auto R) { read_one(0, 0, 0, 0, decltype(R)::value, f0); });

        // With three slots, pair q (A or B [N,K]) lives in slot q % 3; sb =
        // the slot of pair kt / 2.  With two A slots, A pair q in slot q % 2.
        uint32_t sb = 0;
        auto slot3 = [&](uint32_t c) {  // slot of pair kt/2 + c, c <= 4
            const uint32_t s = sb + c, t = s >= 3 ? s - 3 : s;
            return t >= 3 ? t - 3 : t;
        };
        auto bslot = [&](uint32_t c) { return slot3(c) * kBPairBytes; };
        auto aslot = [&](uint32_t c) { return (kASlots == 3 ? slot3(c) : c % 2) * kPairBytes; };
        auto iter = [&](auto U, uint32_t kt) {
            constexpr int u = decltype(U)::value;  // kt % 4 == 0
            const uint32_t j = kt + u;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (BKN) {
                const uint32_t tb = j + 3 < nks ? j + 3 : nks - 1;
                half(f0, f1, aslot(u / 2), u % 2, u * kBStage, 1, std::integral_constant<int, kLoadsB>{},
                     [&](int c) { copy_b(tb, ((u + 3) % S) * kBStage, c); });
            } else {
                // Half (u % 2) of B pair kt/2 + u/2 + 2 (copies 0..kLoadsB-1
                // when j is even, the rest when odd) into its slot, free since
                // the barrier of iteration j-1 (it held pair kt/2 + u/2 - 1).
                const uint32_t q = kt / 2 + u / 2 + 2, qb = q < npairs ? q : npairs - 1;
                const uint32_t dst = bslot(u / 2 + 2);
                half(f0, f1, aslot(u / 2), u % 2, bslot(u / 2) + (u % 2) * 512, 1,
                     std::integral_constant<int, kLoadsB>{}, [&](int c) { copy_b(qb, dst, (u % 2) * kLoadsB + c); });
            }
            __builtin_amdgcn_s_waitcnt(waitcnt_imm(u % 2 == 1 ? kWaitEvenTile : kWaitOddTile, 0));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t bnext = BKN ? ((u + 1) % S) * kBStage : bslot((u + 1) / 2) + ((u + 1) % 2) * 512;
            // Half an A pair, kASlots - 2 pairs further ahead with three
            // slots: j odd, copies 0..3 of pair kt/2 + ca; j even, copies
            // 4..7 (the slot is free since this barrier).
            constexpr int la = kASlots - 2, ca = (u % 2 == 1 ? (u + 3) / 2 : (u + 2) / 2) + la;
            const uint32_t pa = kt / 2 + ca < npairs ? kt / 2 + ca : npairs - 1;
            const uint32_t adst = aslot(ca);
            half(f1, f0, aslot((u + 1) / 2), (u + 1) % 2, bnext, 0, std::integral_constant<int, 4>{},
                 [&](int c) { copy_a(pa, adst, (u % 2 == 1 ? 0 : 4) + c); });
        };
        uint32_t kt = 0;
        for (; kt + S <= nks; kt += S) {
            static_for<S>([&](auto U) { iter(U, kt); });
            sb = sb == 0 ? 2 : sb - 1;  // + 2 pairs
        }
        if (kt < nks) static_for<2>([&](auto U) { iter(U, kt); });  // nks % 4 == 2
        // The trailing copies land before the LDS is reused or released.
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
        __builtin_amdgcn_s_barrier();
    };
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v16i){};
    uint32_t im, in;
    tile_of(blockIdx.x, tm, tn, im, in);
    const uint32_t m0 = im * BM, n0 = in * BN;
    mainloop(m0, n0, 0, nkt);
    if (m0 + BM <= M && n0 + BN <= N && p.ldc <= kFullEpiMaxLdc)
        epilogue_tile_full<EPI, 4, FN, 4>(p, acc, m0 + wm * 128, n0 + wn * (BN / 2), lane);
    else
        epilogue_tile<EPI, 4, FN, 4>(p, acc, m0 + wm * 128 + 4 * (lane / 32), n0 + wn * (BN / 2) + lane % 32, M, N);
}

template <int EPI, bool BKN>
__global__ void __launch_bounds__(256, 1) k_gemm_i8_pairs(const int8_t* __restrict__ A, uint32_t lda,
                                                          const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                          uint32_t N, uint32_t K, EpiParams p) {
    gemm_i8_pairs_tile<EPI, BKN, 256>(A, lda, B, ldb, M, N, K, p);
}
// 256 x 128 tiles (B [N,K]), for grids with too few 256 x 256 tiles.
template <int EPI>
__global__ void __launch_bounds__(256, 1) k_gemm_i8_pairs_n128(const int8_t* __restrict__ A, uint32_t lda,
                                                               const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                               uint32_t N, uint32_t K, EpiParams p) {
    gemm_i8_pairs_tile<EPI, false, 128>(A, lda, B, ldb, M, N, K, p);
}

// --------------------------------------------------- skinny (M <= 16) GEMM

constexpr int kSkWaves = 16, kSkThreads = 64 * kSkWaves, kSkUnroll = 8, kSkPanels = 2;

template <int EPI, bool ALIGNED>
__global__ void __launch_bounds__(kSkThreads) k_gemv_i8_nt(const int8_t* __restrict__ A, uint32_t lda,
                                                           const int8_t* __restrict__ B, uint32_t ldb,
                                                           uint32_t M, uint32_t N, uint32_t K,
                                                           uint32_t k_per_wave, EpiParams p) {
    __shared__ v4i red[kSkWaves][kSkPanels][64];
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t n0 = blockIdx.x * (16 * kSkPanels);
    const uint32_t ra = lane % 16;
    const uint32_t kl = (lane / 16) * 16;
    const uint32_t kbeg = wave * k_per_wave;
    const uint32_t kend = kbeg + k_per_wave < K ? kbeg + k_per_wave : K;

    v4i acc[kSkPanels];
#pragma unroll
    for (int q = 0; q < kSkPanels; q++) acc[q] = (v4i){0, 0, 0, 0};
    for (uint32_t k = kbeg; k < kend; k += 64 * kSkUnroll) {
        v4i a[kSkUnroll], b[kSkPanels][kSkUnroll];
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++) {
            const uint32_t kk = k + u * 64 + kl;
            const bool in = k + u * 64 < kend;
#pragma unroll
            for (int q = 0; q < kSkPanels; q++)
                b[q][u] = in ? load_chunk<ALIGNED>(B, ldb, N, K, n0 + q * 16 + lane % 16, kk) : (v4i){0, 0, 0, 0};
            a[u] = in ? load_chunk<ALIGNED>(A, lda, M, K, ra, kk) : (v4i){0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++)
#pragma unroll
            for (int q = 0; q < kSkPanels; q++)
                acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[q][u], acc[q], 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < kSkPanels; q++) red[wave][q][lane] = acc[q];
    __syncthreads();
    if (wave >= kSkPanels) return;
    const int q = wave;
    v4i s = red[0][q][lane];
#pragma unroll
    for (int w = 1; w < kSkWaves; w++) {
        v4i t = red[w][q][lane];
        s[0] = wrap_add(s[0], t[0]);
        s[1] = wrap_add(s[1], t[1]);
        s[2] = wrap_add(s[2], t[2]);
        s[3] = wrap_add(s[3], t[3]);
    }
    epilogue_store_rows4<EPI>(p, 4 * (lane / 16), n0 + q * 16 + lane % 16, M, N, s);
}

// ---------------------------------------------------- skinny (M <= 16) GEMM

// Y[M,N] = A[M,K] . W[N,K]^T for M <= 16 is a stream of W (64 MiB at
// K = N = 8192) and must run at HBM speed.  Two things decide that on
// MI355X: long contiguous runs per row (an MFMA operand load, 16 rows x 64
// bytes per instruction, reaches only ~4.7 TB/s; whole rows ~6.3 TB/s) and
// ~128 KB in flight per CU.  So W is loaded with plain 16-byte loads laid
// out as 4 rows x 256 contiguous bytes per instruction, landing in VGPRs
// (whose capacity, unlike the LDS's, allows many stages in flight), then
// written into a small LDS buffer of the wave in the MFMA-friendly layout
// and read back as v_mfma_i32_16x16x64_i8 fragments.  A (rows padded to 16
// by repeating row M-1, whose products are never stored) goes the same way,
// so it too moves whole cache lines; A is small and stays in L2.
//
// Block: PANELS 16-row panels of W (the N side of the MFMA), WAVES waves
// splitting K into slices of at most kMaxSlice bytes; a wave walks its
// slice in kMaxStages stages of 256 k-bytes with RS stages in flight
// (kRegStages with one panel, kTwoPanelStages with two), and reuses each A
// fragment for all PANELS panels (halving A's L2 traffic at PANELS = 2).
// The partial tiles of the waves are summed through LDS (int32, wrapping).  The code is straight-line (fully unrolled); loads
// are ordinary, so the compiler's waits are exact, and slices shorter than
// kMaxSlice load clamped (valid) addresses whose products are skipped.  A
// wave's LDS writes and reads execute in order, so no barrier separates a
// stage's write from its reads.  LDS rows are 256 bytes whose 16-byte chunks
// are XOR-swizzled by row (logical chunk c of row r at c ^ r): the 16 lanes
// of a row write one contiguous row, and the fragment reads are
// conflict-free.  Requires 64 <= K, K % 64 == 0, K <= WAVES * kMaxSlice,
// 16-byte aligned operands.
#ifndef RPL_SK_REG_STAGES
#define RPL_SK_REG_STAGES 4
#endif
#ifndef RPL_SK_TWO_PANEL_STAGES
#define RPL_SK_TWO_PANEL_STAGES 3  // M = 16, K = N = 8192: 12.3 us against 12.8 with 4 stages in flight
#endif
#ifndef RPL_SK_ONE_PANEL_MAX_M
#define RPL_SK_ONE_PANEL_MAX_M 8  // larger M: two W panels per block share A (M = 16, K = N = 8192: 12.85 us against 13.24)
#endif
namespace sk {
constexpr int kChunk = 256, kMaxSlice = 2048, kRegStages = RPL_SK_REG_STAGES;
constexpr int kTwoPanelStages = RPL_SK_TWO_PANEL_STAGES;
constexpr int kStageBytes = 16 * kChunk;  // one 16-row panel, one stage
constexpr int kSteps = kChunk / 64;       // MFMA k-steps per stage
constexpr int kMaxStages = kMaxSlice / kChunk;
static_assert(kRegStages >= 1 && kRegStages <= kMaxStages, "stages in flight");
static_assert(kTwoPanelStages >= 1 && kTwoPanelStages <= kMaxStages, "stages in flight");
}  // namespace sk

template <int EPI, int WAVES, int PANELS, int RS = sk::kRegStages>
__global__ void __launch_bounds__(64 * WAVES) k_skinny(const int8_t* __restrict__ A, uint32_t lda,
                                                       const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                       uint32_t N, uint32_t K, uint32_t kpw, EpiParams p) {
    using namespace sk;
    static_assert(RS >= 1 && RS <= kMaxStages, "stages in flight");
    // Per wave: one staging buffer for each W panel and one for A.  A
    // wave's LDS operations execute in issue order, so the next stage's
    // writes cannot overtake this stage's reads.
    constexpr int kBufs = PANELS + 1;
    __shared__ __attribute__((aligned(1024))) int8_t lds_all[WAVES * kBufs * kStageBytes];
    __shared__ v4i red[WAVES][PANELS][64];

    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t n0 = blockIdx.x * 16 * PANELS;
    // Wave w of block b takes K slice (w + b) % WAVES: neighbouring blocks
    // read different parts of A at any moment (the int32 sum over the waves
    // is exact in any order).
    const uint32_t slice = (wave + blockIdx.x) % WAVES;
    const uint32_t kbeg = slice * kpw < K ? slice * kpw : K, kend = kbeg + kpw < K ? kbeg + kpw : K;
    int8_t* const lds = lds_all + wave * kBufs * kStageBytes;
    auto wbuf = [&](int q) { return lds + q * kStageBytes; };
    int8_t* const xbuf = lds + PANELS * kStageBytes;

    // Load instruction i of a stage: rows 4i + lane/16, bytes kb + 16*(lane%16).
    const uint32_t wrow = lane / 16, wchunk = lane % 16;
    auto w_row = [&](int q, uint32_t r) {
        const uint32_t n = n0 + 16 * q + r;
        return B + (uint64_t)(n < N ? n : N - 1) * ldb;
    };
    auto a_row = [&](uint32_t m) { return A + (uint64_t)(m < M ? m : M - 1) * lda; };
    v4i wv[RS][PANELS][4], xv[RS][4];
    auto request = [&](auto T) {
        constexpr int st = decltype(T)::value, r = st % RS;
        uint32_t k = kbeg + st * kChunk + wchunk * 16;
        k = k < kend ? k : kend - 16;  // past the slice: valid bytes, never multiplied
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 4 * i + wrow;
#pragma unroll
            for (int q = 0; q < PANELS; q++)
                wv[r][q][i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w_row(q, row) + k));
            // Row groups at or past M only feed output rows that are never
            // stored: neither loaded nor written to LDS.
            if (4 * i < (int)M) xv[r][i] = *reinterpret_cast<const v4i*>(a_row(row) + k);
        }
    };

    v4i acc[PANELS];
#pragma unroll
    for (int q = 0; q < PANELS; q++) acc[q] = (v4i){0, 0, 0, 0};
    const uint32_t fr = lane % 16;
    static_for<RS>([&](auto T) { request(T); });
    static_for<kMaxStages>([&](auto T) {
        constexpr int st = decltype(T)::value, r = st % RS;
        // Stage st landed (the compiler waits for exactly these loads):
        // write it into this stage's buffers, request stage st + RS,
        // then read the fragments back and multiply.
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 4 * i + wrow, off = row * kChunk + ((wchunk ^ row) * 16);
#pragma unroll
            for (int q = 0; q < PANELS; q++) *reinterpret_cast<v4i*>(wbuf(q) + off) = wv[r][q][i];
            if (4 * i < (int)M) *reinterpret_cast<v4i*>(xbuf + off) = xv[r][i];
        }
        if constexpr (st + RS < kMaxStages) request(std::integral_constant<int, st + RS>{});
        const uint32_t kb = kbeg + st * kChunk;
        const uint32_t left = kend > kb ? (kend - kb) / 64 : 0;
        v4i xs[kSteps];
#pragma unroll
        for (int s = 0; s < kSteps; s++)
            xs[s] = *reinterpret_cast<const v4i*>(xbuf + fr * kChunk + (((4 * s + lane / 16) ^ fr) * 16));
#pragma unroll
        for (int q = 0; q < PANELS; q++) {
            v4i w[kSteps];
#pragma unroll
            for (int s = 0; s < kSteps; s++)
                w[s] = *reinterpret_cast<const v4i*>(wbuf(q) + fr * kChunk + (((4 * s + lane / 16) ^ fr) * 16));
            if (left >= (uint32_t)kSteps) {
#pragma unroll
                for (int s = 0; s < kSteps; s++) acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xs[s], w[s], acc[q], 0, 0, 0);
            } else {
#pragma unroll
                for (int s = 0; s < kSteps; s++)
                    if ((uint32_t)s < left) acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xs[s], w[s], acc[q], 0, 0, 0);
            }
        }
    });
#pragma unroll
    for (int q = 0; q < PANELS; q++) red[wave][q][lane] = acc[q];
    __syncthreads();
    // Wave q < PANELS sums panel q over the waves and stores it.
    if (wave >= (uint32_t)PANELS) return;
    v4i t = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < WAVES; w++) {
        const v4i u = red[w][wave][lane];
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = wrap_add(t[e], u[e]);
    }
    // Result element r of lane l: row 4*(l/16) + r, column l%16 of the panel.
    epilogue_store_rows4<EPI>(p, 4 * (lane / 16), n0 + 16 * wave + lane % 16, M, N, t);
}

// ------------------------------------------- decode-sized (M <= 4) GEMM

// For M <= 4 an MFMA operand would be mostly padding and its lane layout
// (16 rows per load) scatters each HBM load over 16 rows; instead each wave
// streams whole rows of B with v_dot4_i32_i8: one load instruction moves
// 1 KB contiguous (64 lanes x 16 bytes) of one row, and a wave issues all
// the loads of an 8 KB k-slice of its rows before consuming any, so HBM
// latency is paid once per slice.  A (M x K, at most 64 KiB) is staged once
// per block in LDS.  Block: 8 waves x ROWS rows of B.
#ifndef RPL_DV_WAVES
#define RPL_DV_WAVES 8
#endif
constexpr int kDvWaves = RPL_DV_WAVES, kDvThreads = 64 * kDvWaves, kDvSlice = 8;  // 8 x 1 KB per row per slice
constexpr uint32_t kDvMaxA = 64 * 1024;

template <int EPI, int MM, int ROWS, bool ALIGNED>
__global__ void __launch_bounds__(kDvThreads) k_gemv_i8_dot4(const int8_t* __restrict__ A, uint32_t lda,
                                                             const int8_t* __restrict__ B, uint32_t ldb,
                                                             uint32_t M, uint32_t N, uint32_t K, EpiParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t xs[];  // [MM][Kp], Kp = K rounded up to 1024
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t Kp = (K + 1023) / 1024 * 1024;
    const uint32_t n0 = (blockIdx.x * kDvWaves + wave) * ROWS;
    // Issue the first slice of B before staging A, so both are in flight.
    v4i w[ROWS][kDvSlice];
    auto wload = [&](uint32_t k) {
#pragma unroll
        for (int u = 0; u < kDvSlice; u++)
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                const uint32_t kk = k + u * 1024 + lane * 16;
                w[r][u] = kk < Kp ? load_chunk_stream<ALIGNED>(B, ldb, N, K, n0 + r, kk) : (v4i){0, 0, 0, 0};
            }
    };
    wload(0);
    for (uint32_t c = threadIdx.x; c < MM * Kp / 16; c += kDvThreads) {
        const uint32_t m = c / (Kp / 16), k = (c % (Kp / 16)) * 16;
        const v4i v = m < M ? load_chunk<ALIGNED>(A, lda, M, K, m, k) : (v4i){0, 0, 0, 0};
        *reinterpret_cast<v4i*>(&xs[m * Kp + k]) = v;
    }
    __syncthreads();
    int32_t acc[MM][ROWS];
#pragma unroll
    for (int m = 0; m < MM; m++)
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[m][r] = 0;
    for (uint32_t k = 0; k < Kp; k += 1024 * kDvSlice) {
        if (k > 0) wload(k);
#pragma unroll
        for (int u = 0; u < kDvSlice; u++) {
            const uint32_t kk = k + u * 1024 + lane * 16;
            if (kk >= Kp) break;
#pragma unroll
            for (int m = 0; m < MM; m++) {
                const v4i x = *reinterpret_cast<const v4i*>(&xs[m * Kp + kk]);
#pragma unroll
                for (int r = 0; r < ROWS; r++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[m][r] = __builtin_amdgcn_sdot4(x[e], w[r][u][e], acc[m][r], false);
            }
        }
    }
    // Wave-wide int32 sums (wrapping, so any order is exact).
#pragma unroll
    for (int m = 0; m < MM; m++)
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            int32_t v = acc[m][r];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v = wrap_add(v, __shfl_xor(v, off));
            acc[m][r] = v;
        }
    if (lane < (uint32_t)(MM * ROWS)) {
        const uint32_t m = lane / ROWS, r = lane % ROWS;
        int32_t v = 0;
#pragma unroll
        for (int mm = 0; mm < MM; mm++)
#pragma unroll
            for (int rr = 0; rr < ROWS; rr++)
                if (mm == (int)m && rr == (int)r) v = acc[mm][rr];
        if (m < M && n0 + r < N) epilogue_store<EPI>(p, m, n0 + r, v);
    }
}

// ----------------------------------------------------- helpers for gemm_int8

// Bt[n][k] = B[k][n], one 64 x 64-byte tile per block.  Thread (kq, n4)
// loads the 4 dwords B[4kq..4kq+3][4n4..4n4+3] (each load instruction of a
// wave covers 4 rows x 64 contiguous bytes), transposes the 4 x 4 bytes in
// registers, and parks the 4 resulting dwords in an LDS tile laid out
// [n][k-dword] with a 17-dword pitch (conflict-free for this write pattern);
// the tile is then written out row by row, 64 contiguous bytes per 16 lanes.
__global__ void __launch_bounds__(256) k_transpose_i8(const int8_t* __restrict__ B, uint32_t K, uint32_t N,
                                                      int8_t* __restrict__ Bt) {
    __shared__ uint32_t t[64][17];
    const uint32_t k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const uint32_t n4 = threadIdx.x % 16, kq = threadIdx.x / 16;
    const bool full = k0 + 64 <= K && n0 + 64 <= N && N % 4 == 0 && K % 4 == 0 && (((uintptr_t)B) & 3) == 0 &&
                      (((uintptr_t)Bt) & 3) == 0;
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t k = k0 + 4 * kq + i, n = n0 + 4 * n4;
        if (full) {
            d[i] = *reinterpret_cast<const uint32_t*>(B + (uint64_t)k * N + n);
        } else {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; b++)
                if (k < K && n + b < N) v |= (uint32_t)(uint8_t)B[(uint64_t)k * N + n + b] << (8 * b);
            d[i] = v;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t e = ((d[0] >> (8 * j)) & 0xff) | (((d[1] >> (8 * j)) & 0xff) << 8) |
                           (((d[2] >> (8 * j)) & 0xff) << 16) | (((d[3] >> (8 * j)) & 0xff) << 24);
        t[4 * n4 + j][kq] = e;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = threadIdx.x / 16 + 16 * i, c = threadIdx.x % 16;
        const uint32_t n = n0 + r, k = k0 + 4 * c;
        const uint32_t v = t[r][c];
        if (full) {
            *reinterpret_cast<uint32_t*>(Bt + (uint64_t)n * K + k) = v;
        } else if (n < N) {
#pragma unroll
            for (int b = 0; b < 4; b++)
                if (k + b < K) Bt[(uint64_t)n * K + k + b] = (int8_t)(v >> (8 * b));
        }
    }
}

// B [K,N] -> Bt [N,K] for whole 128 x 128 tiles (K, N multiples of 128,
// 16-byte aligned).  Loads move whole 128-byte rows of B into LDS (row
// pitch 144 bytes); the byte transpose is done by ds_read_b64_tr_b8: in each
// group of 16 lanes, output lane 8h+b receives as byte e the byte b of the
// 8-byte piece addressed by lane 2e+h.  Lane 2e+h addresses k-row kb+e at
// column nb+8h, so output lane i gets column nb+i for k-rows kb..kb+7, and
// two reads give it 16 consecutive k-bytes of one column.  Those pieces go
// through the LDS tile again, laid out [n][k], so that the stores write whole
// 128-byte rows of Bt (8 lanes per row): stored straight from the transposed
// reads, every store instruction would touch 64 rows with 16 bytes each,
// and the L2 request rate, not HBM, would set the speed.  Both layouts use a
// 144-byte pitch: the 8 k-rows of a transposed read, and the 16 n-rows a
// lane group writes, fall on distinct LDS banks.
constexpr int kTrTile = 128, kTrPitch = 144;
__global__ void __launch_bounds__(256) k_transpose_i8_tr(const int8_t* __restrict__ B, uint32_t K, uint32_t N,
                                                         int8_t* __restrict__ Bt) {
    // One tile, [k][n] then [n][k]: 18 KB, so 8 blocks fit a CU and keep
    // ~128 KB of loads in flight per CU.
    __shared__ __attribute__((aligned(16))) int8_t s[kTrTile * kTrPitch];
    // Diagonal block order: blocks that run together differ in both n0 (the
    // load side's column) and k0 (the store side's column), so neither side
    // walks one column of rows 8 KB apart.
    const uint32_t nx = N / kTrTile, ny = K / kTrTile, b = blockIdx.x;
    const uint32_t bx = b % nx, by = (b / nx + bx) % ny;
    const uint32_t k0 = by * kTrTile, n0 = bx * kTrTile;
    const uint32_t t = threadIdx.x, lane = t % 64, wave = t / 64;
    v4i v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 32 * i + t / 8, chunk = t % 8;
        v[i] = *reinterpret_cast<const v4i*>(B + (uint64_t)(k0 + row) * N + n0 + 16 * chunk);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 32 * i + t / 8, chunk = t % 8;
        *reinterpret_cast<v4i*>(s + row * kTrPitch + 16 * chunk) = v[i];
    }
    __syncthreads();
    typedef __attribute__((address_space(3))) v2i* lds_v2i;
    const uint32_t g = lane / 16, i = lane % 16;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t idx = wave * 4 + q;
        const uint32_t nb = 64 * (idx % 2) + 16 * g, kb = 16 * (idx / 2);
        const int8_t* a = s + (kb + i / 2) * kTrPitch + nb + 8 * (i % 2);
        const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i)a);
        const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i)(a + 8 * kTrPitch));
        v[q] = (v4i){lo.x, lo.y, hi.x, hi.y};
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t idx = wave * 4 + q;
        const uint32_t nb = 64 * (idx % 2) + 16 * g, kb = 16 * (idx / 2);
        *reinterpret_cast<v4i*>(s + (nb + i) * kTrPitch + kb) = v[q];
    }
    __syncthreads();
#pragma unroll
    for (int i2 = 0; i2 < 4; i2++) {
        const uint32_t row = 32 * i2 + t / 8, chunk = t % 8;
        *reinterpret_cast<v4i*>(Bt + (uint64_t)(n0 + row) * K + k0 + 16 * chunk) =
            *reinterpret_cast<const v4i*>(s + row * kTrPitch + 16 * chunk);
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

// Tile configuration: 256 x 256 tiles on the direct-to-LDS kernel from 3/4
// of a tile per CU (config 3, 2048 x 11008 x 4096: 344 tiles on 256 CUs,
// 123 us against 155 us with 128 x 128 tiles; at half a tile per CU the
// small tiles win), on the register-staged kernel from two tiles per CU;
// else 128 x 128.  RPLHIP_I8_TILE=small|big overrides (tuning sweeps only).
bool use_big_tile(uint32_t M, uint32_t N, bool dma) {
    static const char* env = getenv("RPLHIP_I8_TILE");
    if (env && env[0] == 's') return false;
    if (env && env[0] == 'b') return true;
    const uint64_t tiles = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
    return dma ? 4 * tiles >= 3ull * rplhip::cu_count() : tiles >= 2ull * rplhip::cu_count();
}

// 256 x 128 tiles unless RPLHIP_I8_TILE=small (for A/B timing only).
bool use_half_tile() {
    static const char* env = getenv("RPLHIP_I8_TILE");
    return !(env && env[0] == 's');
}

// One-wave 32 x 32 tiles on small grids unless RPLHIP_I8_SMALL=0 (for A/B
// timing only).
bool use_small_tile() {
    static const char* env = getenv("RPLHIP_I8_SMALL");
    return !(env && env[0] == '0');
}

// The direct-to-LDS kernel serves the big tile unless RPLHIP_I8_DMA=0 (for
// A/B timing only).
bool use_dma() {
    static const char* env = getenv("RPLHIP_I8_DMA");
    return !(env && env[0] == '0');
}

// A copied in k-step pairs (k_gemm_i8_pairs) when K % 128 == 0, unless
// RPLHIP_I8_PAIRS=0 (for A/B timing only).
bool use_pairs(uint32_t K) {
    static const char* env = getenv("RPLHIP_I8_PAIRS");
    return K % (2 * dma::BK) == 0 && !(env && env[0] == '0');
}

// The same epilogue over output columns n1..: the column-indexed inputs
// (bias, B's column sums, per-column scales) and the output start n1 later.
EpiParams shift_cols(EpiParams p, uint32_t n1) {
    if (p.bias) p.bias += n1;
    if (p.rowsum_b) p.rowsum_b += n1;
    if (p.sw && p.sw_per_col) p.sw += n1;
    if (p.out_i32) p.out_i32 += n1;
    if (p.out_f32) p.out_f32 += n1;
    return p;
}

// Rounds of 256 x 256 tiles (one block per CU) that end with a mostly idle
// round: the columns of that round go to a second launch of 256 x 128
// tiles, which run a round in ~0.76 of the big tile's time (2048 x 4096 x
// 4096: 47 us for 256 of them against ~62 us per big round).  Returns the
// width of the big-tile part (a multiple of 256), or 0 to keep one launch.
// Config 3, 2048 x 11008: 344 tiles = 256 + 88 become 256 big tiles on
// N = 8192 and 176 half tiles on the last 2816 columns.
uint32_t balanced_split(uint32_t M, uint32_t N) {
    static const char* env = getenv("RPLHIP_I8_SPLIT");
    if (env && env[0] == '0') return 0;
    const uint64_t C = rplhip::cu_count(), mt = (M + 255) / 256, T = mt * ((N + 255) / 256);
    const uint64_t R = (T + C - 1) / C;
    if (R < 2) return 0;
    const uint64_t n1t = (R - 1) * C / mt;  // tile columns that fill R-1 rounds
    if (n1t == 0 || 256 * n1t >= N) return 0;
    const uint64_t r1 = (mt * n1t + C - 1) / C;
    const uint64_t r2 = (mt * ((N - 256 * n1t + 127) / 128) + C - 1) / C;
    return (double)r1 + 0.76 * (double)r2 < 0.95 * (double)R ? (uint32_t)(256 * n1t) : 0;
}

template <class G, int EPI>
int launch_nt(const int8_t* A, uint32_t lda, const int8_t* B, uint32_t ldb, uint32_t M, uint32_t N, uint32_t K,
              const EpiParams& p, bool al, hipStream_t s) {
    uint64_t tiles = (uint64_t)((M + G::BM - 1) / G::BM) * ((N + G::BN - 1) / G::BN);
    if (tiles > 0x7fffffffull) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "int8 GEMM: %u x %u too large", M, N);
    if (al)
        hipLaunchKernelGGL((k_gemm_i8_nt<G, EPI, true>), dim3((uint32_t)tiles), dim3(G::kThreads), 0, s, A, lda, B,
                           ldb, M, N, K, p);
    else
        hipLaunchKernelGGL((k_gemm_i8_nt<G, EPI, false>), dim3((uint32_t)tiles), dim3(G::kThreads), 0, s, A, lda, B,
                           ldb, M, N, K, p);
    return rplhip::check_launch("int8 GEMM");
}

// K = 0: every accumulator is the empty sum 0 (the k loops of
// src/ops_extended.c:114 and src/rpl_quantization.c:335-345 run no
// iteration), so only the epilogue runs (src/ops_extended.c:119-120, the bias
// add at src/rpl_quantization.c:346-347) and no operand is read.  The GEMM
// kernels' pipelines assume at least one k-step (the pairs kernel two).
template <int EPI>
__global__ void __launch_bounds__(256) k_epilogue_k0(uint32_t M, uint32_t N, EpiParams p) {
    const uint64_t total = (uint64_t)M * N;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256)
        epilogue_store<EPI>(p, (uint32_t)(i / N), (uint32_t)(i % N), 0);
}

// Small grids with short K (config 1, 512^3: 16 tiles of 128 x 128 for 256
// CUs): 32 x 32 tiles, one wave each, on v_mfma_i32_32x32x32_i8 with the
// operand fragments loaded straight from global memory (L2-resident at these
// sizes) into registers.  Lane l reads, for each 32-k step s, bytes
// 32s + 16(l/32) .. +15 of row l%32 of A and of B [N,K]: the MFMA's operand
// layout.  Rows past M / N read the last row (their products are never
// stored); kSmallDepth steps are in flight, the prefetches past the last
// whole step re-read it, so no branch sits around a load and the compiler's
// waits stay exact.  A K % 32 == 16 tail is one more step whose upper k-half
// is zero.  Requires the aligned layout (16-byte rows, K % 16 == 0).
constexpr int kSmallDepth = 8;
constexpr uint32_t kSmallMaxK = 2048;
template <int EPI>
__global__ void __launch_bounds__(64) k_gemm_i8_small(const int8_t* __restrict__ A, uint32_t lda,
                                                      const int8_t* __restrict__ B, uint32_t ldb, uint32_t M,
                                                      uint32_t N, uint32_t K, EpiParams p) {
    const uint32_t lane = threadIdx.x;
    const uint32_t tn = (N + 31) / 32;
    const uint32_t m0 = (blockIdx.x / tn) * 32, n0 = (blockIdx.x % tn) * 32;
    const uint32_t ra = m0 + lane % 32 < M ? m0 + lane % 32 : M - 1;
    const uint32_t rb = n0 + lane % 32 < N ? n0 + lane % 32 : N - 1;
    const int8_t* arow = A + (uint64_t)ra * lda + 16 * (lane / 32);
    const int8_t* brow = B + (uint64_t)rb * ldb + 16 * (lane / 32);
    const uint32_t nkf = K / 32;  // whole 32-k steps
    v16i acc[1][1] = {};
    if (nkf > 0) {
        v4i a[kSmallDepth], b[kSmallDepth];
        auto load = [&](int d, uint32_t st) {
            const uint32_t sc = st < nkf ? st : nkf - 1;
            a[d] = *reinterpret_cast<const v4i*>(arow + 32 * sc);
            b[d] = *reinterpret_cast<const v4i*>(brow + 32 * sc);
        };
#pragma unroll
        for (int d = 0; d < kSmallDepth; d++) load(d, d);
        uint32_t st = 0;
        for (; st + kSmallDepth <= nkf; st += kSmallDepth) {
#pragma unroll
            for (int d = 0; d < kSmallDepth; d++) {
                acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[d], b[d], acc[0][0], 0, 0, 0);
                load(d, st + kSmallDepth + d);
            }
        }
#pragma unroll
        for (int d = 0; d < kSmallDepth; d++)
            if (st + d < nkf) acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[d], b[d], acc[0][0], 0, 0, 0);
    }
    if (K % 32) {
        v4i a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
        if (lane < 32) {
            a = *reinterpret_cast<const v4i*>(arow + 32 * nkf);
            b = *reinterpret_cast<const v4i*>(brow + 32 * nkf);
        }
        acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[0][0], 0, 0, 0);
    }
    epilogue_tile<EPI, 1, 1>(p, acc, m0 + 4 * (lane / 32), n0 + lane % 32, M, N);
}

template <int EPI>
int run_nt(const int8_t* A, uint32_t lda, const int8_t* B, uint32_t ldb, uint32_t M, uint32_t N, uint32_t K,
           const EpiParams& p, hipStream_t s) {
    if (K == 0) {
        const uint64_t blocks = ((uint64_t)M * N + 255) / 256;
        hipLaunchKernelGGL((k_epilogue_k0<EPI>), dim3((uint32_t)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s,
                           M, N, p);
        return rplhip::check_launch("int8 GEMM, K = 0");
    }
    bool al = K % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && aligned16(A) && aligned16(B);
    const uint32_t Kp = (K + 1023) / 1024 * 1024;
    const bool skinny_ok = al && K >= 64 && K % 64 == 0 && K <= 8 * sk::kMaxSlice;
    if (M <= 4 && !skinny_ok && (uint64_t)4 * Kp <= kDvMaxA) {
        size_t lds = (size_t)(M <= 1 ? 1 : M <= 2 ? 2 : 4) * Kp;
#define RPL_DV(MM, ROWS)                                                                                           \
    do {                                                                                                           \
        dim3 grid((N + kDvWaves * ROWS - 1) / (kDvWaves * ROWS));                                                  \
        if (al)                                                                                                    \
            hipLaunchKernelGGL((k_gemv_i8_dot4<EPI, MM, ROWS, true>), grid, dim3(kDvThreads), lds, s, A, lda, B,  \
                               ldb, M, N, K, p);                                                                   \
        else                                                                                                       \
            hipLaunchKernelGGL((k_gemv_i8_dot4<EPI, MM, ROWS, false>), grid, dim3(kDvThreads), lds, s, A, lda, B, \
                               ldb, M, N, K, p);                                                                   \
    } while (0)
        if (M <= 1)
            RPL_DV(1, 1);
        else if (M <= 2)
            RPL_DV(2, 1);
        else
            RPL_DV(4, 2);
#undef RPL_DV
        return rplhip::check_launch("decode int8 GEMM");
    }
    if (M <= 16 && skinny_ok) {
        // 4 waves when their K slices fit kMaxSlice, else 8; with 4 waves,
        // two panels per block (A fragments shared) when M >
        // RPL_SK_ONE_PANEL_MAX_M (8 waves x 2 panels would spill).
        const uint32_t waves = K <= 4 * sk::kMaxSlice ? 4 : 8;
        uint32_t kpw = (K + waves - 1) / waves;
        kpw = (kpw + 63) / 64 * 64;
        const bool two = waves == 4 && M > RPL_SK_ONE_PANEL_MAX_M;
        const dim3 grid(two ? (N + 31) / 32 : (N + 15) / 16);
        if constexpr (RPL_SK_ONE_PANEL_MAX_M < 16) {  // two panels are only reachable below M = 16
            if (two) {
                hipLaunchKernelGGL((k_skinny<EPI, 4, 2, sk::kTwoPanelStages>), grid, dim3(256), 0, s, A, lda, B, ldb, M, N, K, kpw, p);
                return rplhip::check_launch("skinny int8 GEMM");
            }
        }
        if (waves == 4)
            hipLaunchKernelGGL((k_skinny<EPI, 4, 1>), grid, dim3(256), 0, s, A, lda, B, ldb, M, N, K, kpw, p);
        else
            hipLaunchKernelGGL((k_skinny<EPI, 8, 1>), grid, dim3(512), 0, s, A, lda, B, ldb, M, N, K, kpw, p);
        return rplhip::check_launch("skinny int8 GEMM");
    }
    if (M <= 16) {
        // Split K over the block's waves in 64-byte steps.
        uint32_t kpw = (K + kSkWaves - 1) / kSkWaves;
        kpw = (kpw + 63) / 64 * 64;
        dim3 grid((N + 16 * kSkPanels - 1) / (16 * kSkPanels));
        if (al)
            hipLaunchKernelGGL((k_gemv_i8_nt<EPI, true>), grid, dim3(kSkThreads), 0, s, A, lda, B, ldb, M, N, K,
                               kpw, p);
        else
            hipLaunchKernelGGL((k_gemv_i8_nt<EPI, false>), grid, dim3(kSkThreads), 0, s, A, lda, B, ldb, M, N, K,
                               kpw, p);
        return rplhip::check_launch("skinny int8 GEMM");
    }
    // Odd shapes (byte-wise loads) always take the small tile: the big one
    // has no registers to spare for them.
    const bool dma_ok =
        al && K % dma::BK == 0 && (uint64_t)M * lda < (1ull << 31) && (uint64_t)N * ldb < (1ull << 31) && use_dma();
    const uint64_t mt = (M + dma::BM - 1) / dma::BM;
    if (al && use_big_tile(M, N, dma_ok)) {
        const uint32_t n1 = dma_ok ? balanced_split(M, N) : 0;
        if (n1) {
            // Columns [0, n1) on big tiles, [n1, N) on 256 x 128 tiles.
            const EpiParams p2 = shift_cols(p, n1);
            const uint32_t tiles1 = (uint32_t)(mt * (n1 / 256)), tiles2 = (uint32_t)(mt * ((N - n1 + 127) / 128));
            if (use_pairs(K))
                hipLaunchKernelGGL((k_gemm_i8_pairs<EPI, false>), dim3(tiles1), dim3(dma::kThreads), 0, s, A, lda,
                                   B, ldb, M, n1, K, p);
            else
                hipLaunchKernelGGL((k_gemm_i8_nt_dma<EPI, 256>), dim3(tiles1), dim3(dma::kThreads), 0, s, A, lda, B,
                                   ldb, M, n1, K, p);
            if (use_pairs(K))
                hipLaunchKernelGGL((k_gemm_i8_pairs_n128<EPI>), dim3(tiles2), dim3(dma::kThreads), 0, s, A,
                                   lda, B + (uint64_t)n1 * ldb, ldb, M, N - n1, K, p2);
            else
                hipLaunchKernelGGL((k_gemm_i8_nt_dma<EPI, 128>), dim3(tiles2), dim3(dma::kThreads), 0, s, A, lda,
                                   B + (uint64_t)n1 * ldb, ldb, M, N - n1, K, p2);
            return rplhip::check_launch("int8 GEMM (balanced halves)");
        }
        if (dma_ok) {
            const uint64_t tiles = mt * ((N + 255) / 256);
            if (use_pairs(K))
                hipLaunchKernelGGL((k_gemm_i8_pairs<EPI, false>), dim3((uint32_t)tiles), dim3(dma::kThreads),
                                   0, s, A, lda, B, ldb, M, N, K, p);
            else
                hipLaunchKernelGGL((k_gemm_i8_nt_dma<EPI, 256>), dim3((uint32_t)tiles), dim3(dma::kThreads), 0, s, A,
                                   lda, B, ldb, M, N, K, p);
            return rplhip::check_launch("int8 GEMM");
        }
        return launch_nt<CfgBig, EPI>(A, lda, B, ldb, M, N, K, p, al, s);
    }
    // Too few 256 x 256 tiles: 256 x 128 ones on the same kernel when they
    // give at least 3/4 of a tile per CU (config 3, 2048 x 4096 x 4096: 256).
    const uint64_t tiles_half = mt * ((N + 127) / 128);
    if (dma_ok && use_half_tile() && 4 * tiles_half >= 3ull * rplhip::cu_count()) {
        if (use_pairs(K))
            hipLaunchKernelGGL((k_gemm_i8_pairs_n128<EPI>), dim3((uint32_t)tiles_half), dim3(dma::kThreads), 0,
                               s, A, lda, B, ldb, M, N, K, p);
        else
            hipLaunchKernelGGL((k_gemm_i8_nt_dma<EPI, 128>), dim3((uint32_t)tiles_half), dim3(dma::kThreads), 0, s, A,
                               lda, B, ldb, M, N, K, p);
        return rplhip::check_launch("int8 GEMM");
    }
    // 128 x 128 tiles for fewer than a quarter of the CUs and a short K: one
    // wave per 32 x 32 tile instead (512^3: 256 waves against 16 blocks,
    // 7.45 -> 3.69 us; at 1024^2, 64 tiles, the 128 x 128 kernel is faster).
    const uint64_t tiles128 = (uint64_t)((M + 127) / 128) * ((N + 127) / 128);
    const uint64_t tiles32 = (uint64_t)((M + 31) / 32) * ((N + 31) / 32);
    if (al && K <= kSmallMaxK && 4 * tiles128 < rplhip::cu_count() && use_small_tile()) {
        hipLaunchKernelGGL((k_gemm_i8_small<EPI>), dim3((uint32_t)tiles32), dim3(64), 0, s, A, lda, B, ldb, M, N, K,
                           p);
        return rplhip::check_launch("int8 GEMM (small grid)");
    }
    return launch_nt<CfgSmall, EPI>(A, lda, B, ldb, M, N, K, p, al, s);
}

// B stored [K][N] (gemm_int8's layout, ldb = N) read in place by the
// direct-to-LDS kernel: shapes that take its 256 x 256 tile, N % 16 == 0.
// RPLHIP_I8_KN=0 sends them through the transposed copy instead (for A/B
// timing only).
bool kn_ok(const int8_t* A, const int8_t* B, uint32_t M, uint32_t N, uint32_t K) {
    static const char* env = getenv("RPLHIP_I8_KN");
    if (env && env[0] == '0') return false;
    if (M <= 16 || K == 0 || K % dma::BK || N % 16 || !aligned16(A) || !aligned16(B))
        return false;
    if ((uint64_t)M * K >= (1ull << 31) || (uint64_t)K * N >= (1ull << 31)) return false;
    const uint64_t tiles = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
    return use_dma() && use_big_tile(M, N, true) && tiles <= 0x7fffffffull;
}

template <int EPI>
int launch_kn(const int8_t* A, const int8_t* B, uint32_t M, uint32_t N, uint32_t K, const EpiParams& p,
              hipStream_t s) {
    const uint32_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
    if (use_pairs(K))
        hipLaunchKernelGGL((k_gemm_i8_pairs<EPI, true>), dim3(tiles), dim3(dma::kThreads), 0, s, A, K, B, N,
                           M, N, K, p);
    else
        hipLaunchKernelGGL((k_gemm_i8_nt_dma<EPI, 256, true>), dim3(tiles), dim3(dma::kThreads), 0, s, A, K, B, N, M,
                           N, K, p);
    return rplhip::check_launch("int8 GEMM ([K][N] B)");
}

// True (and *inv = 1/sc) when sc = +-2^k is a normal float whose reciprocal
// is exactly representable: then x / sc and x * (1/sc) are both the
// correctly rounded value of the same real number, for every x (overflow,
// subnormal results, infinities and NaN included).
bool exact_reciprocal(float sc, float* inv) {
    if (!isfinite(sc) || sc == 0.0f) return false;
    int e;
    const float m = frexpf(fabsf(sc), &e);  // |sc| = m * 2^e, m in [0.5, 1)
    if (m != 0.5f || e - 1 < -126) return false;
    *inv = ldexpf(sc > 0 ? 1.0f : -1.0f, 1 - e);
    return true;
}

// True when every requantized value ((float)acc * sa) * sb of a K-long int8
// dot product (|acc| <= K * 128 * 128) is finite and below 2^30 in
// magnitude, so the x86 range test of the conversion can never fire.
bool requant_in_range(uint32_t K, float sa, float sb) {
    if (!isfinite(sa) || !isfinite(sb)) return false;
    const double bound = (double)K * 16384.0 * fabs((double)sa) * fabs((double)sb) * (1.0 + 1e-6);
    return bound < 1073741824.0;
}

int transpose_b(const int8_t* B, uint32_t K, uint32_t N, int8_t* Bt, hipStream_t s) {
    const uint64_t tr_tiles = (uint64_t)(N / kTrTile) * (K / kTrTile);
    if (K % kTrTile == 0 && N % kTrTile == 0 && aligned16(B) && aligned16(Bt) && tr_tiles <= 0x7fffffffull) {
        hipLaunchKernelGGL(k_transpose_i8_tr, dim3((uint32_t)tr_tiles), dim3(256), 0, s, B, K, N, Bt);
        return rplhip::check_launch("int8 transpose");
    }
    dim3 grid((N + 63) / 64, (K + 63) / 64);
    if (grid.y > 65535) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "int8 transpose: K=%u too large", K);
    hipLaunchKernelGGL(k_transpose_i8, grid, dim3(256), 0, s, B, K, N, Bt);
    return rplhip::check_launch("int8 transpose");
}

// gemm_int8's B is read in place when the kernel can (the column sums of a
// zero point of B come from the transposed copy).
bool gemm_int8_reads_b_in_place(const int8_t* A, const int8_t* B, uint32_t M, uint32_t N, uint32_t K, int32_t za) {
    return za == 0 && kn_ok(A, B, M, N, K);
}

// Device scratch bytes of one gemm_int8 call: the transposed copy of B
// (unless B is read in place), then A's row sums (zb != 0) and B's column
// sums (za != 0).
size_t gemm_int8_scratch_bytes(bool kn, uint32_t M, uint32_t N, uint32_t K, int32_t za, int32_t zb) {
    const size_t bt = kn ? 0 : ((size_t)K * N + 15) / 16 * 16;
    return bt + sizeof(int32_t) * ((za ? (size_t)N : 0) + (zb ? (size_t)M : 0)) + 16;
}

// gemm_int8 on scratch `ws` of at least gemm_int8_scratch_bytes(kn, ...).
int gemm_int8_run(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K, float sa,
                  float sb, float sc, int32_t za, int32_t zb, bool kn, void* ws, hipStream_t s) {
    const size_t bt_bytes = kn ? 0 : ((size_t)K * N + 15) / 16 * 16;
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
    int st = RPLHIP_OK;
    if (K && !kn) st = transpose_b(B, K, N, Bt, s);
    if (!st && zb && K) {
        p.rowsum_a = sum_ptr;
        sum_ptr += M;
        hipLaunchKernelGGL(k_rowsum_i8, dim3(M), dim3(256), 0, s, A, M, K, (int32_t*)p.rowsum_a);
        st = rplhip::check_launch("int8 row sums");
    }
    if (!st && za && K) {
        p.rowsum_b = sum_ptr;
        hipLaunchKernelGGL(k_rowsum_i8, dim3(N), dim3(256), 0, s, Bt, N, K, (int32_t*)p.rowsum_b);
        st = rplhip::check_launch("int8 column sums");
    }
    if (st) return st;
    if (za == 0 && zb == 0 && sc == 1.0f && requant_in_range(K, sa, sb))
        return kn ? launch_kn<kRequantUnit>(A, B, M, N, K, p, s) : run_nt<kRequantUnit>(A, K, Bt, K, M, N, K, p, s);
    if (za == 0 && zb == 0 && exact_reciprocal(sc, &p.inv_sc))
        return kn ? launch_kn<kRequantPow2>(A, B, M, N, K, p, s) : run_nt<kRequantPow2>(A, K, Bt, K, M, N, K, p, s);
    return kn ? launch_kn<kRequant>(A, B, M, N, K, p, s) : run_nt<kRequant>(A, K, Bt, K, M, N, K, p, s);
}

// Static scratch of rplhip_gemm_int8_noalloc.  Device code never names the
// array: kernels get its address as an argument, like a workspace.  On the
// host `scratch` is only a stand-in symbol (a kernel given it would fault);
// the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int kMaxDevices = 64;
pthread_mutex_t g_scratch_mu = PTHREAD_MUTEX_INITIALIZER;
void* g_scratch_ptr[kMaxDevices];

}  // namespace

static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

namespace {

// Device address of `scratch` on the current device (looked up on the
// device's first call, then cached).
int noalloc_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return rplhip::fail(RPLHIP_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "device %d out of range", dev);
    pthread_mutex_lock(&g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            pthread_mutex_unlock(&g_scratch_mu);
            return rplhip::fail(RPLHIP_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        }
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    pthread_mutex_unlock(&g_scratch_mu);
    return RPLHIP_OK;
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
    const bool kn = gemm_int8_reads_b_in_place(A, B, M, N, K, za);
    void* ws = nullptr;
    int st = ws_alloc(&ws, gemm_int8_scratch_bytes(kn, M, N, K, za, zb), s);
    if (st) return st;
    st = gemm_int8_run(A, B, C, M, N, K, sa, sb, sc, za, zb, kn, ws, s);
    ws_free(ws, s);
    return st;
}

// gemm_int8 with its scratch (the transposed copy of B and the zero-point
// sums) in the library's static device array instead of a workspace
// allocation: no hipMalloc, hipFree or allocating library call.  Every call
// on a device shares that device's array, so calls that overlap in time on
// one device (different streams, no ordering between them) race; calls on
// one stream are ordered and safe.  Every byte of scratch a call reads is
// written by the same call first, so nothing needs clearing.
int rplhip_gemm_int8_noalloc(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K,
                             float sa, float sb, float sc, int32_t za, int32_t zb, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!C || (K && (!A || !B))) return fail(RPLHIP_ERR_INVALID, "rplhip_gemm_int8_noalloc: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    const bool kn = gemm_int8_reads_b_in_place(A, B, M, N, K, za);
    const size_t need = gemm_int8_scratch_bytes(kn, M, N, K, za, zb);
    if (need > kNoAllocScratchBytes)
        return fail(RPLHIP_ERR_UNSUPPORTED,
                    "rplhip_gemm_int8_noalloc: %u x %u x %u (za %d, zb %d) needs %zu bytes of scratch, more than "
                    "the %zu-byte static scratch",
                    M, N, K, za, zb, need, kNoAllocScratchBytes);
    void* ws = nullptr;
    int st = noalloc_scratch(&ws);
    if (st) return st;
    return gemm_int8_run(A, B, C, M, N, K, sa, sb, sc, za, zb, kn, ws, as_stream(stream));
}

int rplhip_gemm_int8_dequant(const int8_t* A, const float* a_scale, int a_per_row, const int8_t* B,
                             const float* b_scale, int b_per_col, float* Y, uint32_t M, uint32_t N, uint32_t K,
                             rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!Y || !a_scale || !b_scale || (K && (!A || !B)))
        return fail(RPLHIP_ERR_INVALID, "rplhip_gemm_int8_dequant: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    EpiParams p = {};
    p.sx = a_scale;
    p.sw = b_scale;
    p.sx_per_row = a_per_row;
    p.sw_per_col = b_per_col;
    p.out_f32 = Y;
    p.ldc = N;
    if (kn_ok(A, B, M, N, K)) return launch_kn<kDequant>(A, B, M, N, K, p, s);
    void* ws = nullptr;
    int st = ws_alloc(&ws, ((size_t)K * N + 15) / 16 * 16 + 16, s);
    if (st) return st;
    if (K) st = transpose_b(B, K, N, (int8_t*)ws, s);
    if (!st) st = run_nt<kDequant>(A, K, (const int8_t*)ws, K, M, N, K, p, s);
    ws_free(ws, s);
    return st;
}

}  // extern "C"
