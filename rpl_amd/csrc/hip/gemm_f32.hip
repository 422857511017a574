// FP32 GEMM on gfx950 f32 MFMA (v_mfma_f32_16x16x4_f32):
//   C = alpha * op(A) * op(B) + beta * C, row-major, all four transposes.
//
// Block tile 128 x 128 x 32, 4 waves (2 x 2), each wave a 64 x 64 sub-tile of
// 4 x 4 MFMA blocks.  Tiles are copied HBM -> registers -> LDS unchanged
// (128-bit loads along each operand's contiguous dimension, double-buffered
// LDS), and every MFMA operand is then fetched with one ds_read_b128 that
// serves four MFMAs:
//   * an operand stored k-contiguous (A as [M,K], B as [N,K]) is read as
//     4 consecutive k of one row   -> the 4 k-substeps of a 16-k slice;
//   * an operand stored row-contiguous (A as [K,M], B as [K,N]) is read as
//     4 consecutive rows of one k  -> the 4 MFMA blocks of the wave, whose
//     rows are then interleaved (block f owns rows f, f+4, f+8, ...).
// Both give lane l the k index 4*(l/16) + s of substep s, so A and B agree.
// With B stored [K,N] the interleaved output columns make every lane own 4
// consecutive columns, so C is read and written with 128-bit accesses.
#include <stdlib.h>

#include "mfma_pipe.h"
#include "rplhip_internal.h"

namespace {

using rplhip::lds_ptr;
using rplhip::static_for;
using rplhip::swz;
using rplhip::uniform_rsrc;
using rplhip::waitcnt_imm;

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kThreads = 256;
constexpr int TM = 64, TN = 64;  // wave tile
constexpr int FM = 4, FN = 4;    // 16x16 MFMA blocks per wave tile
constexpr int kPadK = BK + 4;    // pitch (floats) of a k-contiguous LDS tile
constexpr int kPadR = BM + 4;    // pitch (floats) of a row-contiguous LDS tile
constexpr int kTileFloats = (BM * kPadK > BK * kPadR) ? BM * kPadK : BK * kPadR;
constexpr int kLoads = BM * BK / 4 / kThreads;  // float4 per thread per operand

// Operand geometry: a tile of R rows (M or N) by BK k-values.  KCONTIG: the
// global matrix is [R_total, K] (k contiguous), else [K, R_total].
template <bool KCONTIG, bool VEC>
struct Operand {
    const float* __restrict__ base;
    uint32_t ld, rows, K;

    // Chunk c of the tile -> (tile row, tile k) of its first element.
    __device__ __forceinline__ static void chunk_pos(uint32_t c, uint32_t& r, uint32_t& k) {
        if (KCONTIG) {
            r = c / (BK / 4);
            k = (c % (BK / 4)) * 4;
        } else {
            k = c / (BM / 4);
            r = (c % (BM / 4)) * 4;
        }
    }

    __device__ __forceinline__ float4 load(uint32_t r0, uint32_t k0, uint32_t c) const {
        uint32_t r, k;
        chunk_pos(c, r, k);
        r += r0;
        k += k0;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (KCONTIG) {
            if (r >= rows) return v;
            const float* p = base + (uint64_t)r * ld + k;
            if (VEC) {
                if (k < K) v = *reinterpret_cast<const float4*>(p);
            } else {
                v.x = k + 0 < K ? p[0] : 0.f;
                v.y = k + 1 < K ? p[1] : 0.f;
                v.z = k + 2 < K ? p[2] : 0.f;
                v.w = k + 3 < K ? p[3] : 0.f;
            }
        } else {
            if (k >= K) return v;
            const float* p = base + (uint64_t)k * ld + r;
            if (VEC) {
                if (r < rows) v = *reinterpret_cast<const float4*>(p);
            } else {
                v.x = r + 0 < rows ? p[0] : 0.f;
                v.y = r + 1 < rows ? p[1] : 0.f;
                v.z = r + 2 < rows ? p[2] : 0.f;
                v.w = r + 3 < rows ? p[3] : 0.f;
            }
        }
        return v;
    }

    __device__ __forceinline__ static void store(float* s, uint32_t c, float4 v) {
        uint32_t r, k;
        chunk_pos(c, r, k);
        if (KCONTIG)
            *reinterpret_cast<float4*>(&s[r * kPadK + k]) = v;
        else
            *reinterpret_cast<float4*>(&s[k * kPadR + r]) = v;
    }

    // Fragments for one 16-k slice (kh): frag[f][s] is the value this lane
    // feeds MFMA block f at substep s.
    __device__ __forceinline__ static void frags(const float* s, uint32_t wofs, uint32_t lane, int kh,
                                                 float frag[4][4]) {
        const uint32_t kg = lane / 16, li = lane % 16;
        if (KCONTIG) {
#pragma unroll
            for (int f = 0; f < 4; f++) {
                float4 v = *reinterpret_cast<const float4*>(&s[(wofs + f * 16 + li) * kPadK + kh * 16 + 4 * kg]);
                frag[f][0] = v.x;
                frag[f][1] = v.y;
                frag[f][2] = v.z;
                frag[f][3] = v.w;
            }
        } else {
#pragma unroll
            for (int sub = 0; sub < 4; sub++) {
                float4 v = *reinterpret_cast<const float4*>(&s[(kh * 16 + 4 * kg + sub) * kPadR + wofs + li * 4]);
                frag[0][sub] = v.x;
                frag[1][sub] = v.y;
                frag[2][sub] = v.z;
                frag[3][sub] = v.w;
            }
        }
    }

    // Tile-relative row of MFMA block f, in-block index i (0..15).
    __device__ __forceinline__ static uint32_t row_of(uint32_t wofs, int f, uint32_t i) {
        return KCONTIG ? wofs + f * 16 + i : wofs + i * 4 + f;
    }
};

// SPLIT: block (tile, blockIdx.y) multiplies only k in [blockIdx.y * kps,
// +kps) (kps a multiple of BK) and stores the raw partial tile to
// C + blockIdx.y * M * ldc (a workspace; alpha, beta are applied by
// k_splitk_reduce).  Batches: blockIdx.z selects matrices A + z*sA,
// B + z*sB, C + z*sC.  read_c = 0 drops the read of C (beta is then
// ignored); rplhip_sgemm always reads it, as the reference does.
template <bool TA, bool TB, bool VEC, bool SPLIT>
__global__ void __launch_bounds__(kThreads, 2) k_sgemm(uint32_t M, uint32_t N, uint32_t K, float alpha,
                                                       const float* __restrict__ A, uint32_t lda,
                                                       const float* __restrict__ B, uint32_t ldb, float beta,
                                                       float* __restrict__ C, uint32_t ldc, uint32_t kps,
                                                       uint64_t sA, uint64_t sB, uint64_t sC, int read_c) {
    A += blockIdx.z * sA;
    B += blockIdx.z * sB;
    C += blockIdx.z * sC;
    using OpA = Operand<!TA, VEC>;
    using OpB = Operand<TB, VEC>;
    __shared__ __attribute__((aligned(16))) float As[2][kTileFloats];
    __shared__ __attribute__((aligned(16))) float Bs[2][kTileFloats];

    const OpA opa{A, lda, M, K};
    const OpB opb{B, ldb, N, K};
    const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const uint32_t wm = (wave / 2) * TM, wn = (wave % 2) * TN;
    // 1-D tile grid in the XCD-aware grouped order (A and B panels shared
    // by the CUs of an XCD stay in its L2).
    uint32_t im, in;
    rplhip::tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, im, in);
    const uint32_t m0 = im * BM, n0 = in * BN;

    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    float4 ra[kLoads], rb[kLoads];
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < kLoads; i++) ra[i] = opa.load(m0, k0, tid + i * kThreads);
#pragma unroll
        for (int i = 0; i < kLoads; i++) rb[i] = opb.load(n0, k0, tid + i * kThreads);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kLoads; i++) OpA::store(As[buf], tid + i * kThreads, ra[i]);
#pragma unroll
        for (int i = 0; i < kLoads; i++) OpB::store(Bs[buf], tid + i * kThreads, rb[i]);
    };

    const uint32_t kbeg = SPLIT ? blockIdx.y * kps : 0;
    const uint32_t kend = SPLIT && kbeg + kps < K ? kbeg + kps : K;
    if (SPLIT) C += (uint64_t)blockIdx.y * M * ldc;
    const uint32_t nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    gload(kbeg);
    sstore(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kbeg + (kt + 1) * BK);
#pragma unroll
        for (int kh = 0; kh < BK / 16; kh++) {
            float fa[4][4], fb[4][4];
            OpA::frags(As[buf], wm, lane, kh, fa);
            OpB::frags(Bs[buf], wn, lane, kh, fb);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane owns column lane%16 and rows 4*(lane/16)+r of each block.
    const uint32_t li = lane % 16, rg = 4 * (lane / 16);
    if (SPLIT) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    uint32_t m = m0 + OpA::row_of(wm, i, rg + r);
                    uint32_t n = n0 + OpB::row_of(wn, j, li);
                    if (m < M && n < N) C[(uint64_t)m * ldc + n] = acc[i][j][r];
                }
    } else if (!TB && VEC) {
        // Interleaved columns: block j holds column li*4 + j -> 4 consecutive
        // columns per lane, one float4 read-modify-write per (i, r).  All of
        // the lane's C reads are issued before its first store: with a store
        // between them the compiler cannot prove the next read's address
        // different (it does not know ldc >= N, which the entry points
        // check), so each read would wait for the one before (16 round trips).
        float4 cv[FM][4];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t m = m0 + OpA::row_of(wm, i, rg + r), n = n0 + wn + li * 4;
                cv[i][r] = read_c && m < M && n < N ? *reinterpret_cast<const float4*>(&C[(uint64_t)m * ldc + n])
                                                    : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                uint32_t m = m0 + OpA::row_of(wm, i, rg + r);
                uint32_t n = n0 + wn + li * 4;
                if (m >= M || n >= N) continue;
                float4 c = cv[i][r];
                c.x = alpha * acc[i][0][r] + beta * c.x;
                c.y = alpha * acc[i][1][r] + beta * c.y;
                c.z = alpha * acc[i][2][r] + beta * c.z;
                c.w = alpha * acc[i][3][r] + beta * c.w;
                *reinterpret_cast<float4*>(&C[(uint64_t)m * ldc + n]) = c;
            }
    } else {
        // C reads first, then the stores (as above; 64 round trips per lane
        // otherwise).
        float cv[FM][FN][4];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t m = m0 + OpA::row_of(wm, i, rg + r), n = n0 + OpB::row_of(wn, j, li);
                    cv[i][j][r] = read_c && m < M && n < N ? C[(uint64_t)m * ldc + n] : 0.0f;
                }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    uint32_t m = m0 + OpA::row_of(wm, i, rg + r);
                    uint32_t n = n0 + OpB::row_of(wn, j, li);
                    if (m < M && n < N)
                        C[(uint64_t)m * ldc + n] = alpha * acc[i][j][r] + (read_c ? beta * cv[i][j][r] : 0.0f);
                }
    }
}

// ------------------------------------------ direct-to-LDS kernel (big grids)
//
// For grids with several 256 x 256 tiles per CU (8192^3: four).  Block tile
// 256 x 256 x 16, 4 waves (2 x 2) of 128 x 128, one wave per SIMD, on
// v_mfma_f32_32x32x2f32 (4096 flops per 64-cycle issue) with the 16 x 16
// accumulator registers per 32 x 32 block in AGPRs.  The load unit copies
// the tiles HBM -> LDS itself (buffer_load_dword x4 ... lds, 1 KB per
// instruction) into a ring of S stages; one barrier per 16-k tile, between
// its two 8-k halves.  A 16-k tile is 64 flops per byte of LDS traffic, so
// each stage carries 8192 MFMA cycles per wave: latency hides easily.
//
// Operand kinds, both 16 KB per stage:
//  * k-contiguous (A as [M,K], B as [N,K]): 256 rows of 64 bytes, the four
//    16-byte k-chunks of row r at slot c ^ swz(r); one copy instruction moves
//    16 rows (lane l: row l/4, chunk (l%4) ^ swz(row) chosen at the source).
//    Fragment read for half t: lane l reads chunk l/32 + 2t of row l%32 of
//    each 32-row block -> floats k = 4(l/32) + 8t + s, s = 0..3: one 128-bit
//    read serves the block's four substeps.
//  * row-contiguous (A as [K,M], B as [K,N]): 16 k-rows of 1 KB; one copy
//    instruction moves one k-row.  The wave's four blocks interleave their
//    rows (block f owns tile rows wofs + 4c + f), so lane l reading floats
//    wofs + 4(l%32) .. +3 of k-row 4(l/32) + 8t + s gets substep s of all
//    four blocks in one 128-bit read.
// Both kinds give lane l the same k for (t, s), so A and B agree.  Rows past
// the matrix are clamped to the last row and columns to the last 4 (their
// products are never stored), so no copy leaves the operand.
// Requires K % 16 == 0, 16-byte aligned bases, ld % 4 == 0, N % 4 == 0
// (and M % 4 == 0 for A as [K,M]), operands below 2 GiB.
#ifndef RPL_F32_STAGES
#define RPL_F32_STAGES 4
#endif
namespace fd {
constexpr int BM = 256, BN = 256, BK = 16, S = RPL_F32_STAGES, kThreads = 256;
constexpr int kTileBytes = BM * BK * 4;  // one operand of one stage: 16 KB
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kLoads = 4;                // 1 KB copies per wave per operand per tile
constexpr int kVmPerTile = 2 * kLoads;
static_assert(S >= 3 && S * kStageBytes <= 160 * 1024, "LDS ring must fit 160 KB");

// One operand of the tile: KC = k-contiguous in memory.
template <bool KC>
struct Op {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff[kLoads];
    uint32_t kstep;  // bytes to advance one 16-k tile
    uint32_t fofs;   // lane's fragment offset within the operand's LDS tile (half 0)

    // X: [rows_total, K] (KC) or [K, rows_total]; r0 = first tile row.
    __device__ __forceinline__ void init(const float* X, uint32_t ld, uint32_t rows_total, uint32_t K, uint32_t r0,
                                         uint32_t wave, uint32_t lane, uint32_t wofs) {
        const uint32_t valid = rows_total - r0 < (uint32_t)BM ? rows_total - r0 : BM;
        if (KC) {
            rsrc = uniform_rsrc(X + (uint64_t)r0 * ld, valid * ld * 4);
#pragma unroll
            for (int i = 0; i < kLoads; i++) {
                const uint32_t r = wave * 64 + i * 16 + lane / 4;
                voff[i] = (r < valid ? r : valid - 1) * ld * 4 + ((lane % 4) ^ swz(r)) * 16;
            }
            kstep = BK * 4;
            const uint32_t fr = lane % 32;
            fofs = (wofs + fr) * 64 + ((lane / 32) ^ swz(fr)) * 16;
        } else {
            rsrc = uniform_rsrc(X + r0, (uint32_t)(((uint64_t)(K - 1) * ld + valid) * 4));
            const uint32_t c = 4 * lane < valid - 4 ? 4 * lane : valid - 4;
#pragma unroll
            for (int i = 0; i < kLoads; i++) voff[i] = (wave * kLoads + i) * ld * 4 + c * 4;
            kstep = BK * ld * 4;
            fofs = (4 * (lane / 32)) * (BM * 4) + (wofs + 4 * (lane % 32)) * 4;
        }
    }

    __device__ __forceinline__ void issue(uint32_t kt, char* st, uint32_t wave) const {
#pragma unroll
        for (int i = 0; i < kLoads; i++) {
            char* dst = KC ? st + (wave * 64 + i * 16) * 64 : st + (wave * kLoads + i) * (BM * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr)dst, 16, voff[i], kt * kstep, 0, 0);
        }
    }

    // Fragment registers of half t: KC: x[b] = block b, substeps 0..3;
    // row-contiguous: x[s] = substep s, blocks 0..3.
    __device__ __forceinline__ void frags(const char* st, int t, v4f (&x)[4]) const {
        // KC: chunk l/32 + 2t sits at slot (l/32 ^ swz) ^ 2t, i.e. the half-0
        // offset with bit 5 flipped (rows are 64-byte aligned).
        const uint32_t base = KC ? (fofs ^ (32u * t)) : fofs + 8 * t * (BM * 4);
#pragma unroll
        for (int q = 0; q < 4; q++)
            x[q] = *reinterpret_cast<const v4f*>(st + base + (KC ? q * 32 * 64 : q * (BM * 4)));
    }

    // Operand of block f at substep s.
    __device__ __forceinline__ static float val(const v4f (&x)[4], int f, int s) { return KC ? x[f][s] : x[s][f]; }

    // Tile-relative row (within the wave's 128) of block f, block-local row i.
    __device__ __forceinline__ static uint32_t row(int f, uint32_t i) { return KC ? f * 32 + i : 4 * i + f; }
};
}  // namespace fd

template <bool TA, bool TB>
__global__ void __launch_bounds__(256, 1) k_sgemm_dma(uint32_t M, uint32_t N, uint32_t K, float alpha,
                                                      const float* __restrict__ A, uint32_t lda,
                                                      const float* __restrict__ B, uint32_t ldb, float beta,
                                                      float* __restrict__ C, uint32_t ldc, int read_c) {
    using fd::BK;
    using fd::BM;
    using fd::BN;
    using fd::kLoads;
    using fd::kStageBytes;
    using fd::kTileBytes;
    using fd::kVmPerTile;
    using fd::S;
    using OpA = fd::Op<!TA>;
    using OpB = fd::Op<TB>;
    __shared__ __attribute__((aligned(1024))) char smem[S * kStageBytes];

    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t wm = wave / 2, wn = wave % 2;
    uint32_t im, in;
    rplhip::tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, im, in);
    const uint32_t m0 = im * BM, n0 = in * BN;
    OpA opa;
    OpB opb;
    opa.init(A, lda, M, K, m0, wave, lane, wm * 128);
    opb.init(B, ldb, N, K, n0, wave, lane, wn * 128);

    auto issue_a = [&](uint32_t kt, uint32_t stage) { opa.issue(kt, smem + stage * kStageBytes, wave); };
    auto issue_b = [&](uint32_t kt, uint32_t stage) { opb.issue(kt, smem + stage * kStageBytes + kTileBytes, wave); };
    auto issue = [&](uint32_t kt, uint32_t stage) {
        issue_a(kt, stage);
        issue_b(kt, stage);
    };
    // Wait until this wave's copies of tile kt+1 have landed, given that
    // `later` whole tiles were issued after it.
    auto wait_after = [&](uint32_t later) {
        static_for<S - 1>([&](auto Cn) {
            constexpr int c = decltype(Cn)::value;
            if (later == (uint32_t)c) __builtin_amdgcn_s_waitcnt(waitcnt_imm(c * kVmPerTile, 0));
        });
    };
    struct F {
        v4f a[4], b[4];
    };
    auto fload = [&](uint32_t stage, int t, F& f) {
        const char* st = smem + stage * kStageBytes;
        opa.frags(st, t, f.a);
        opb.frags(st + kTileBytes, t, f.b);
    };
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (v16f){};
    auto mma = [&](const F& f) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(OpA::val(f.a, i, s), OpB::val(f.b, j, s),
                                                                     acc[i][j], 0, 0, 0);
    };
    // Pin each half's order: the 8 fragment reads early, one between
    // MFMA pairs, then the tile copies, so no MFMA waits on a read issued
    // just before it.
    auto pin = [&](auto copies) {
        static_for<8>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        });
        static_for<decltype(copies)::value>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // HBM -> LDS copy
        });
    };

    const uint32_t nk = K / BK;
    static_for<S - 1>([&](auto T) {
        constexpr int t = decltype(T)::value;
        if (t < nk) issue(t, t);
    });
    wait_after(nk - 1 < (uint32_t)(S - 2) ? nk - 1 : S - 2);
    __builtin_amdgcn_s_barrier();
    F f0, f1;
    fload(0, 0, f0);

    // Iteration kt: request tile kt+S-1 (A copies in the first half, B in
    // the second) into the stage tile kt-1 left, read tile kt's second half
    // while multiplying its first, wait for tile kt+1 and barrier, read tile
    // kt+1's first half while multiplying kt's second.
    constexpr int kLaterSteady = (S - 3) * kVmPerTile + kLoads;
    uint32_t kt = 0;
    for (; kt + 2 * S - 1 <= nk; kt += S) {
        static_for<S>([&](auto U) {
            constexpr int u = decltype(U)::value;
            __builtin_amdgcn_sched_barrier(0);
            issue_a(kt + u + S - 1, (u + S - 1) % S);
            fload(u, 1, f1);
            mma(f0);
            pin(std::integral_constant<int, kLoads>{});
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(waitcnt_imm(kLaterSteady, 0));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            issue_b(kt + u + S - 1, (u + S - 1) % S);
            fload((u + 1) % S, 0, f0);
            mma(f1);
            pin(std::integral_constant<int, kLoads>{});
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    for (; kt < nk; kt++) {
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        fload(kt % S, 1, f1);
        mma(f0);
        const uint32_t last = kt + S - 1 < nk - 1 ? kt + S - 1 : nk - 1;
        wait_after(last > kt + 1 ? last - kt - 1 : 0);
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < nk) fload((kt + 1) % S, 0, f0);
        mma(f1);
    }

    // Epilogue.  Result register r of lane l in block (i, j) is block-local
    // row 8(r/4) + 4(l/32) + r%4 and column l%32.
    // Per row block i, all C reads are issued before the first store: with a
    // store between two reads the compiler cannot prove the second address
    // different (ldc >= N is checked by the entry points, not known here) and
    // each read would wait for the one before (64 round trips per lane).
    const uint32_t mw = m0 + wm * 128, nw = n0 + wn * 128;
    const bool full = m0 + BM <= M && n0 + BN <= N;
    auto row_m = [&](int i, int r) { return mw + OpA::row(i, 8 * (r / 4) + 4 * (lane / 32) + r % 4); };
    if constexpr (!TB) {
        if (full && read_c) {
            // Interior tile, in units of 8 rows (half a row block): unit
            // u+1's C reads are issued before unit u's stores, so each
            // unit's reads wait only for the stores of the unit two back
            // (stores count in vmcnt).  The units are distinct rows of C
            // (ldc >= N).  Two units in flight keep 64 VGPRs of C, as one
            // whole row block does.
            const uint32_t n = nw + 4 * (lane % 32);
            float4 cv[2][8];
            auto load_c = [&](auto U) {
                constexpr int u = decltype(U)::value;
#pragma unroll
                for (int r = 0; r < 8; r++)
                    cv[u % 2][r] =
                        *reinterpret_cast<const float4*>(C + (uint64_t)row_m(u / 2, 8 * (u % 2) + r) * ldc + n);
            };
            load_c(std::integral_constant<int, 0>{});
            static_for<8>([&](auto U) {
                constexpr int u = decltype(U)::value, i = u / 2;
                if constexpr (u + 1 < 8) load_c(std::integral_constant<int, u + 1>{});
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    const int rr = 8 * (u % 2) + r;
                    float4 c = cv[u % 2][r];
                    c.x = alpha * acc[i][0][rr] + beta * c.x;
                    c.y = alpha * acc[i][1][rr] + beta * c.y;
                    c.z = alpha * acc[i][2][rr] + beta * c.z;
                    c.w = alpha * acc[i][3][rr] + beta * c.w;
                    *reinterpret_cast<float4*>(C + (uint64_t)row_m(i, rr) * ldc + n) = c;
                }
            });
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (!TB) {
            // Interleaved columns: block j holds column 4(l%32) + j.
            const uint32_t n = nw + 4 * (lane % 32);
            float4 cv[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = row_m(i, r);
                const bool ok = full || (m < M && n + 3 < N);
                cv[r] = read_c && ok ? *reinterpret_cast<const float4*>(C + (uint64_t)m * ldc + n)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = row_m(i, r);
                if (!(full || (m < M && n + 3 < N))) continue;
                float4 c = cv[r];
                c.x = alpha * acc[i][0][r] + beta * c.x;
                c.y = alpha * acc[i][1][r] + beta * c.y;
                c.z = alpha * acc[i][2][r] + beta * c.z;
                c.w = alpha * acc[i][3][r] + beta * c.w;
                *reinterpret_cast<float4*>(C + (uint64_t)m * ldc + n) = c;
            }
        } else {
            // Two halves of 8 rows, 32 reads in flight each (all 64 at once
            // spilled scalar registers).
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float cv[8][4];
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    const uint32_t m = row_m(i, 8 * h + r);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t n = nw + j * 32 + lane % 32;
                        cv[r][j] = read_c && (full || (m < M && n < N)) ? C[(uint64_t)m * ldc + n] : 0.0f;
                    }
                }
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    const uint32_t m = row_m(i, 8 * h + r);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t n = nw + j * 32 + lane % 32;
                        if (full || (m < M && n < N))
                            C[(uint64_t)m * ldc + n] =
                                alpha * acc[i][j][8 * h + r] + (read_c ? beta * cv[r][j] : 0.0f);
                    }
                }
            }
        }
    }
}

// C = alpha * sum_s W[s] + beta * C over the split partials W[s] ([M, N],
// ld N), summed in split order (deterministic).  With a bias, also
// out2 = C + bias[n] (linear_forward's broadcast add, a separately rounded
// float add as src/rpl_core.c:112-120 does it).
__global__ void __launch_bounds__(256) k_splitk_reduce(const float* __restrict__ W, uint32_t splits, uint32_t M,
                                                       uint32_t N, float alpha, float beta, float* __restrict__ C,
                                                       uint32_t ldc, int read_c, const float* __restrict__ bias,
                                                       float* __restrict__ out2) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)M * N) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    // Loads in batches of 8 (one chain of dependent loads was latency-bound:
    // ~9 us for 32 splits); the additions keep split order.
    const uint64_t stride = (uint64_t)M * N;
    float sum = W[i];
    uint32_t s = 1;
    for (; s + 8 <= splits; s += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = W[(uint64_t)(s + j) * stride + i];
#pragma unroll
        for (int j = 0; j < 8; j++) sum += v[j];
    }
    for (; s < splits; s++) sum += W[(uint64_t)s * stride + i];
    float* cp = &C[(uint64_t)m * ldc + n];
    const float c = alpha * sum + (read_c ? beta * *cp : 0.0f);
    *cp = c;
    if (bias) out2[(uint64_t)m * ldc + n] = c + bias[n];
}

bool aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

// ----------------------------------------- wave-split kernel (small grids)
//
// For products whose 128 x 128 tiles leave most CUs idle (the MLP's
// 4096 x 128 x 784 forward product, its 128 x 784 x 4096 and 10 x 128 x 4096
// weight gradients).  One block per (16 FM) x 64 output tile and K range; each
// of its 4 waves multiplies the WHOLE tile over a quarter of the block's K
// range, loading its operands from global memory straight into registers (no
// LDS and no barrier in the k loop), P steps of 16 k in flight.  The waves'
// partial tiles are then added in LDS in wave order, so the result does not
// depend on timing.  A K range split over several blocks (nsplit > 1) writes
// raw partial tiles W[split] ([M, N], ld N) for k_splitk_reduce; otherwise the
// block applies alpha, beta and the bias itself, as k_splitk_reduce does.
#ifndef RPL_WS_WAVES
#define RPL_WS_WAVES 4
#endif
#ifndef RPL_WS_PREFETCH
#define RPL_WS_PREFETCH 3
#endif
namespace wsk {
constexpr int kWaves = RPL_WS_WAVES, kThreads = 64 * kWaves, FN = 4, BN = 16 * FN, P = RPL_WS_PREFETCH;

// One operand of a wave's 16-k step.  KC: stored [rows, K] (k contiguous),
// else [K, rows].  F = the wave's MFMA blocks along this operand.  v[f][s] is
// what this lane feeds block f at substep s, whose k is k0 + 4 (lane / 16) + s
// for every lane group (so A and B agree).  Addresses are clamped into the
// matrix: a row past `rows` only feeds output rows or columns that are never
// stored, and a k past K only prefetched steps that are never multiplied, so
// the k loop takes the values as loaded (a select or a branch per load made
// the compiler wait for each load at once).  MASK zeroes k >= K, for the one
// partial step at the end of K.
template <bool KC, int F>
struct WaveOp {
    const float* __restrict__ base;
    uint32_t ld, rows, K;

    template <bool MASK>
    __device__ __forceinline__ void load(uint32_t r0, uint32_t k0, uint32_t lane, float v[F][4]) const {
        const uint32_t g = lane / 16, li = lane % 16;
        if (KC) {
            // block f, in-block row li = tile row 16 f + li; 4 consecutive k
            // (K % 4 == 0)
            const uint32_t k = k0 + 4 * g, kc = k < K ? k : K - 4;
#pragma unroll
            for (int f = 0; f < F; f++) {
                const uint32_t r = r0 + 16 * f + li, rc = r < rows ? r : rows - 1;
                const float4 x = *reinterpret_cast<const float4*>(base + (uint64_t)rc * ld + kc);
                const bool ok = !MASK || k < K;
                v[f][0] = ok ? x.x : 0.f;
                v[f][1] = ok ? x.y : 0.f;
                v[f][2] = ok ? x.z : 0.f;
                v[f][3] = ok ? x.w : 0.f;
            }
        } else {
            // k-row k0 + 4g + s; F consecutive rows F li .. F li + F - 1, row
            // F li + f being block f's in-block row li (rows % F == 0)
            const uint32_t r = r0 + F * li, rc = r < rows ? r : rows - F;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint32_t k = k0 + 4 * g + s, kc = k < K ? k : K - 1;
                const bool ok = !MASK || k < K;
                const float* p = base + (uint64_t)kc * ld + rc;
                if (F == 4) {
                    const float4 x = *reinterpret_cast<const float4*>(p);
                    v[0][s] = ok ? x.x : 0.f;
                    v[1 % F][s] = ok ? x.y : 0.f;
                    v[2 % F][s] = ok ? x.z : 0.f;
                    v[3 % F][s] = ok ? x.w : 0.f;
                } else if (F == 2) {
                    const float2 x = *reinterpret_cast<const float2*>(p);
                    v[0][s] = ok ? x.x : 0.f;
                    v[1 % F][s] = ok ? x.y : 0.f;
                } else {
                    const float x = *p;
                    v[0][s] = ok ? x : 0.f;
                }
            }
        }
    }

    // Tile-relative row of block f's in-block row i.
    __device__ __forceinline__ static uint32_t row_of(int f, uint32_t i) { return KC ? 16 * f + i : F * i + f; }
};

template <bool TA, bool TB, int FM, bool SPLIT>
__global__ void __launch_bounds__(kThreads) k_sgemm_ws(uint32_t M, uint32_t N, uint32_t K, float alpha,
                                                       const float* __restrict__ A, uint32_t lda,
                                                       const float* __restrict__ B, uint32_t ldb, float beta,
                                                       float* __restrict__ C, uint32_t ldc, int read_c,
                                                       const float* __restrict__ bias, float* __restrict__ out2,
                                                       uint32_t tiles_m, uint32_t tiles_n, uint32_t spb) {
    constexpr int BM = 16 * FM, kPitch = BN + 4;
    using OpA = WaveOp<!TA, FM>;
    using OpB = WaveOp<TB, FN>;
    __shared__ __attribute__((aligned(16))) float red[kWaves][BM * kPitch];

    // Blocks b, b + 8, b + 16, ... run on one XCD: give them consecutive
    // (split, tile m, tile n) so that they share operand panels in its L2.
    const uint32_t total = gridDim.x, full = total / 8 * 8;
    uint32_t lin = blockIdx.x < full ? (blockIdx.x % 8) * (full / 8) + blockIdx.x / 8 : blockIdx.x;
    const uint32_t tn = lin % tiles_n;
    lin /= tiles_n;
    const uint32_t tm = lin % tiles_m, sp = lin / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t steps = (K + 15) / 16;
    const uint32_t b0 = sp * spb, b1 = b0 + spb < steps ? b0 + spb : steps;
    const uint32_t spw = (b1 - b0 + kWaves - 1) / kWaves;
    const uint32_t w0 = b0 + wave * spw < b1 ? b0 + wave * spw : b1;
    const uint32_t w1 = w0 + spw < b1 ? w0 + spw : b1;
    const uint32_t kbeg = 16 * w0, kend = 16 * w1 < K ? 16 * w1 : K;
    const int n = (int)(w1 - w0);

    const OpA opa{A, lda, M, K};
    const OpB opb{B, ldb, N, K};
    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    float a[P][FM][4], b[P][FN][4];
    auto load = [&](int slot, int t) {
        opa.template load<false>(m0, kbeg + 16 * t, lane, a[slot]);
        opb.template load<false>(n0, kbeg + 16 * t, lane, b[slot]);
    };
    auto step = [&](int slot) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[slot][i][s], b[slot][j][s], acc[i][j], 0, 0, 0);
    };
    // Full steps in a ring of P slots; prefetches past them are never
    // multiplied, so the loop body needs no condition.  A partial last step
    // (K % 16 != 0, the last wave with steps) is loaded again masked.
    const bool partial = n > 0 && (kend & 15) != 0;
    const int nf = n - (partial ? 1 : 0);
#pragma unroll
    for (int u = 0; u < P; u++) load(u, u);
    int t = 0;
    for (; t + P <= nf; t += P) {
#pragma unroll
        for (int u = 0; u < P; u++) {
            // Kept in this order: slot u's refill issued right after its
            // multiplies, so the loads complete in slot order and the wait
            // before slot u + 1 leaves 2 slots' loads in flight.
            step(u);
            __builtin_amdgcn_sched_barrier(0);
            load(u, t + u + P);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < P - 1; u++)
        if (nf - t > u) step(u);
    if (partial) {
        opa.template load<true>(m0, kbeg + 16 * nf, lane, a[0]);
        opb.template load<true>(n0, kbeg + 16 * nf, lane, b[0]);
        step(0);
    }

    // Partial tiles into LDS; then each thread adds the four waves' values of
    // 4 consecutive columns, in wave order.
    const uint32_t g = lane / 16, li = lane % 16;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                red[wave][OpA::row_of(i, 4 * g + r) * kPitch + OpB::row_of(j, li)] = acc[i][j][r];
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < (uint32_t)(BM * BN / 4); e += kThreads) {
        const uint32_t row = e / (BN / 4), col = 4 * (e % (BN / 4));
        const uint32_t m = m0 + row, nn = n0 + col;
        if (m >= M || nn >= N) continue;  // N % 4 == 0: a column group is all in or all out
        float4 sum = *reinterpret_cast<const float4*>(&red[0][row * kPitch + col]);
#pragma unroll
        for (int w = 1; w < kWaves; w++) {
            const float4 x = *reinterpret_cast<const float4*>(&red[w][row * kPitch + col]);
            sum.x += x.x;
            sum.y += x.y;
            sum.z += x.z;
            sum.w += x.w;
        }
        if (SPLIT) {
            *reinterpret_cast<float4*>(&C[(uint64_t)sp * M * N + (uint64_t)m * N + nn]) = sum;
        } else {
            float* cp = &C[(uint64_t)m * ldc + nn];
            float4 c = read_c ? *reinterpret_cast<const float4*>(cp) : make_float4(0.f, 0.f, 0.f, 0.f);
            c.x = alpha * sum.x + (read_c ? beta * c.x : 0.0f);
            c.y = alpha * sum.y + (read_c ? beta * c.y : 0.0f);
            c.z = alpha * sum.z + (read_c ? beta * c.z : 0.0f);
            c.w = alpha * sum.w + (read_c ? beta * c.w : 0.0f);
            *reinterpret_cast<float4*>(cp) = c;
            if (bias) {
                const float4 bv = *reinterpret_cast<const float4*>(&bias[nn]);
                *reinterpret_cast<float4*>(&out2[(uint64_t)m * ldc + nn]) =
                    make_float4(c.x + bv.x, c.y + bv.y, c.z + bv.z, c.w + bv.w);
            }
        }
    }
}

// Steps of 16 k per wave below which a K split over blocks is not worth its
// partial tiles.
constexpr uint32_t kMinWaveSteps = 4;

template <bool TA, bool TB, int FM>
int launch_fm(uint32_t M, uint32_t N, uint32_t K, float alpha, const float* A, uint32_t lda, const float* B,
              uint32_t ldb, float beta, float* C, uint32_t ldc, hipStream_t s, int read_c, const float* bias,
              float* out2) {
    const uint32_t tiles_m = (M + 16 * FM - 1) / (16 * FM), tiles_n = (N + BN - 1) / BN;
    const uint64_t tiles = (uint64_t)tiles_m * tiles_n;
    const uint32_t steps = (K + 15) / 16;
    uint64_t ns = rplhip::cu_count() / tiles;
    const uint64_t cap = steps / (kWaves * kMinWaveSteps);
    if (ns > cap) ns = cap;
    if (ns < 1) ns = 1;
    const uint32_t spb = (uint32_t)((steps + ns - 1) / ns);
    ns = spb ? (steps + spb - 1) / spb : 1;
    if (ns < 1) ns = 1;
    if (tiles * ns > 0x7fffffffull) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "sgemm: %u x %u too large", M, N);
    const dim3 grid((uint32_t)(tiles * ns));
    if (ns == 1) {
        hipLaunchKernelGGL((k_sgemm_ws<TA, TB, FM, false>), grid, dim3(kThreads), 0, s, M, N, K, alpha, A, lda, B, ldb,
                           beta, C, ldc, read_c, bias, out2, tiles_m, tiles_n, spb);
        return rplhip::check_launch("sgemm (wave split)");
    }
    void* ws = nullptr;
    int st = rplhip::ws_alloc(&ws, (size_t)ns * M * N * sizeof(float), s);
    if (st) return st;
    hipLaunchKernelGGL((k_sgemm_ws<TA, TB, FM, true>), grid, dim3(kThreads), 0, s, M, N, K, 1.0f, A, lda, B, ldb,
                       0.0f, (float*)ws, N, 0, nullptr, nullptr, tiles_m, tiles_n, spb);
    st = rplhip::check_launch("sgemm (wave split)");
    if (!st) {
        const uint64_t total = (uint64_t)M * N;
        hipLaunchKernelGGL(k_splitk_reduce, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, (const float*)ws,
                           (uint32_t)ns, M, N, alpha, beta, C, ldc, read_c, bias, out2);
        st = rplhip::check_launch("sgemm (wave split reduction)");
    }
    rplhip::ws_free(ws, s);
    return st;
}

bool aligned(const void* p, uintptr_t bytes) { return (((uintptr_t)p) % bytes) == 0; }

// Whether an operand suits WaveOp<KC, F>'s vector loads.
bool operand_ok(bool kc, int f, const float* p, uint32_t ld, uint32_t rows, uint32_t K) {
    return kc ? aligned(p, 16) && ld % 4 == 0 && K % 4 == 0 : aligned(p, 4 * f) && ld % f == 0 && rows % f == 0;
}

// Tile height: the largest of 64 / 32 / 16 rows whose tiles fill the CUs
// without a K split; else 64 rows (16 or 32 for short M).  Returns -1, having
// launched nothing, when the operands do not suit the kernel's vector
// accesses.
template <bool TA, bool TB>
int launch(uint32_t M, uint32_t N, uint32_t K, float alpha, const float* A, uint32_t lda, const float* B,
           uint32_t ldb, float beta, float* C, uint32_t ldc, hipStream_t s, int read_c, const float* bias,
           float* out2) {
    const uint64_t tn = (N + BN - 1) / BN, cu = rplhip::cu_count();
    int fm = M <= 16 ? 1 : M <= 32 ? 2 : 4;
    if ((M + 63) / 64 * tn < cu) {
        if ((M + 31) / 32 * tn >= cu)
            fm = 2;
        else if ((M + 15) / 16 * tn >= cu)
            fm = 1;
    }
    if (!operand_ok(!TA, fm, A, lda, M, K) || !operand_ok(TB, FN, B, ldb, N, K) || !aligned(C, 16) || ldc % 4 ||
        N % 4 || (bias && (!aligned(bias, 16) || !aligned(out2, 16))))
        return -1;
    if (fm == 1) return launch_fm<TA, TB, 1>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c, bias, out2);
    if (fm == 2) return launch_fm<TA, TB, 2>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c, bias, out2);
    return launch_fm<TA, TB, 4>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c, bias, out2);
}
}  // namespace wsk

// K splits for a grid of `tiles` tiles: enough blocks to fill the CUs twice,
// each split at least RPL_F32_MIN_KSPLIT long (a multiple of BK); 1 = no
// split.  Measured minimum lengths 256 / 128 / 64: config 0 (512^3) 27.0 /
// 19.2 / 17.3 us, config 2's MLP step 219 / 202 / 210 us.
#ifndef RPL_F32_MIN_KSPLIT
#define RPL_F32_MIN_KSPLIT 128
#endif
uint32_t k_splits(uint64_t tiles, uint32_t K) {
    const uint64_t want = 2ull * rplhip::cu_count();
    if (tiles >= want / 2 || K < 2 * RPL_F32_MIN_KSPLIT) return 1;
    uint64_t s = (want + tiles - 1) / tiles;
    const uint64_t cap = K / RPL_F32_MIN_KSPLIT;
    return (uint32_t)(s < cap ? s : cap);
}

// Small products (K <= 256, M*N*K <= 2^23; the MLP's 4096 x 128 x 10 and
// 4096 x 10 x 128): one thread per output element on the VALU.  The 128 x 128
// MFMA tile gives them 32 blocks, which leave most CUs idle (~18 us each).
// The operation order is src/rpl_core.c:208-213's: sum = fma(a, b, sum) over
// k in order, then C = fma(alpha, sum, beta * C) (GCC's contraction of
// alpha*sum + beta*C), so these outputs equal the reference's bit for bit.
// V4 (A as [M,K] and B as [N,K], 16-byte aligned rows): the same fma chain
// fed by 128-bit loads, 8 of each in flight (the scalar loads left the
// 4096 x 10 x 128 product latency-bound).
template <bool TA, bool TB, bool V4>
__global__ void __launch_bounds__(256) k_sgemm_valu(uint32_t M, uint32_t N, uint32_t K, float alpha,
                                                    const float* __restrict__ A, uint32_t lda,
                                                    const float* __restrict__ B, uint32_t ldb, float beta,
                                                    float* __restrict__ C, uint32_t ldc, int read_c,
                                                    const float* __restrict__ bias, float* __restrict__ out2) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)M * N) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    float sum = 0.0f;
    uint32_t k0 = 0;
    if constexpr (V4) {
        static_assert(!TA && TB, "V4 reads both operands along k");
        const float4* a4 = reinterpret_cast<const float4*>(A + (uint64_t)m * lda);
        const float4* b4 = reinterpret_cast<const float4*>(B + (uint64_t)n * ldb);
#pragma unroll 8
        for (uint32_t q = 0; q < K / 4; q++) {
            const float4 a = a4[q], b = b4[q];
            sum = __builtin_fmaf(a.x, b.x, sum);
            sum = __builtin_fmaf(a.y, b.y, sum);
            sum = __builtin_fmaf(a.z, b.z, sum);
            sum = __builtin_fmaf(a.w, b.w, sum);
        }
        k0 = K / 4 * 4;
    }
#pragma unroll 8
    for (uint32_t k = k0; k < K; k++) {
        const float a = TA ? A[(uint64_t)k * lda + m] : A[(uint64_t)m * lda + k];
        const float b = TB ? B[(uint64_t)n * ldb + k] : B[(uint64_t)k * ldb + n];
        sum = __builtin_fmaf(a, b, sum);
    }
    float* cp = &C[(uint64_t)m * ldc + n];
    const float c = __builtin_fmaf(alpha, sum, read_c ? beta * *cp : 0.0f);
    *cp = c;
    if (bias) out2[(uint64_t)m * ldc + n] = c + bias[n];  // separately rounded, as src/rpl_core.c:112-120
}

// The same chain for A as [M,K] and B as [N,K] with few columns (the MLP's
// 4096 x 10 x 128): the block's 256 outputs need only rows m0..m1 of A and
// all N rows of B, which it first copies into LDS with 128-bit loads (one
// round of memory latency instead of one per 32 k), then every thread runs
// its fma chain from LDS.  Rows are padded to K + 4 floats, so the rows read
// together fall on distinct banks.
__global__ void __launch_bounds__(256) k_sgemm_valu_lds(uint32_t M, uint32_t N, uint32_t K, float alpha,
                                                        const float* __restrict__ A, uint32_t lda,
                                                        const float* __restrict__ B, uint32_t ldb, float beta,
                                                        float* __restrict__ C, uint32_t ldc, int read_c,
                                                        const float* __restrict__ bias, float* __restrict__ out2) {
    extern __shared__ __attribute__((aligned(16))) float lds_ab[];
    const uint32_t pitch = K + 4, k4 = K / 4;
    const uint64_t i0 = (uint64_t)blockIdx.x * 256, total = (uint64_t)M * N;
    const uint64_t ilast = i0 + 255 < total ? i0 + 255 : total - 1;
    const uint32_t m0 = (uint32_t)(i0 / N), rows_a = (uint32_t)(ilast / N) - m0 + 1;
    float* as = lds_ab;
    float* bs = lds_ab + (uint64_t)rows_a * pitch;
    for (uint32_t c = threadIdx.x; c < rows_a * k4; c += 256) {
        const uint32_t r = c / k4, q = c % k4;
        *reinterpret_cast<float4*>(&as[r * pitch + 4 * q]) =
            *reinterpret_cast<const float4*>(A + (uint64_t)(m0 + r) * lda + 4 * q);
    }
    for (uint32_t c = threadIdx.x; c < N * k4; c += 256) {
        const uint32_t r = c / k4, q = c % k4;
        *reinterpret_cast<float4*>(&bs[r * pitch + 4 * q]) =
            *reinterpret_cast<const float4*>(B + (uint64_t)r * ldb + 4 * q);
    }
    __syncthreads();
    const uint64_t i = i0 + threadIdx.x;
    if (i >= total) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    const float4* a4 = reinterpret_cast<const float4*>(&as[(m - m0) * pitch]);
    const float4* b4 = reinterpret_cast<const float4*>(&bs[n * pitch]);
    float sum = 0.0f;
#pragma unroll 8
    for (uint32_t q = 0; q < k4; q++) {
        const float4 a = a4[q], b = b4[q];
        sum = __builtin_fmaf(a.x, b.x, sum);
        sum = __builtin_fmaf(a.y, b.y, sum);
        sum = __builtin_fmaf(a.z, b.z, sum);
        sum = __builtin_fmaf(a.w, b.w, sum);
    }
    float* cp = &C[(uint64_t)m * ldc + n];
    const float c = __builtin_fmaf(alpha, sum, read_c ? beta * *cp : 0.0f);
    *cp = c;
    if (bias) out2[(uint64_t)m * ldc + n] = c + bias[n];  // separately rounded, as src/rpl_core.c:112-120
}
// LDS the block needs, or 0 when the shape does not suit k_sgemm_valu_lds.
size_t valu_lds_bytes(uint32_t N, uint32_t K) {
    if (K == 0 || K % 4 || N > 64) return 0;
    const size_t rows = 256 / N + 2 + N;
    const size_t bytes = rows * (K + 4) * sizeof(float);
    return bytes <= 64 * 1024 ? bytes : 0;
}

constexpr uint32_t kValuMaxK = 256;
constexpr uint64_t kValuMaxWork = 1ull << 23;

// The same products with a longer K (the MLP's dW2, 10 x 128 x 4096): block
// row y sums k in [y * kps, +kps) into the workspace W[y] ([M, N], ld N), and
// k_splitk_reduce adds the slices in order.  (The VALU path does two loads per
// fma, so it stays within kValuMaxWork; larger products keep the MFMA tiles.)
constexpr uint32_t kValuSlice = 64, kValuMaxSlices = 256;
template <bool TA, bool TB>
__global__ void __launch_bounds__(256) k_sgemm_valu_split(uint32_t M, uint32_t N, uint32_t K,
                                                          const float* __restrict__ A, uint32_t lda,
                                                          const float* __restrict__ B, uint32_t ldb,
                                                          float* __restrict__ W, uint32_t kps) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)M * N) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    const uint32_t k0 = blockIdx.y * kps, k1 = k0 + kps < K ? k0 + kps : K;
    float sum = 0.0f;
#pragma unroll 8
    for (uint32_t k = k0; k < k1; k++) {
        const float a = TA ? A[(uint64_t)k * lda + m] : A[(uint64_t)m * lda + k];
        const float b = TB ? B[(uint64_t)n * ldb + k] : B[(uint64_t)k * ldb + n];
        sum = __builtin_fmaf(a, b, sum);
    }
    W[(uint64_t)blockIdx.y * M * N + i] = sum;
}

// read_c = 0: C is written without being read (beta ignored); the result
// equals that of read_c = 1 over C = 0 bit for bit (alpha*x + 0.0f).
// bias (ldc == N): also out2 = C + bias[n], fused into the last pass of the
// VALU and split-K paths, a broadcast add after the others.
template <bool TA, bool TB>
int launch(uint32_t M, uint32_t N, uint32_t K, float alpha, const float* A, uint32_t lda, const float* B,
           uint32_t ldb, float beta, float* C, uint32_t ldc, hipStream_t s, int read_c = 1,
           const float* bias = nullptr, float* out2 = nullptr) {
    // 128-bit paths need the contiguous extents and leading dimensions to be
    // multiples of 4 floats and 16-byte aligned bases.
    bool vec = aligned16(A) && aligned16(B) && aligned16(C) && lda % 4 == 0 && ldb % 4 == 0 &&
               ldc % 4 == 0 && N % 4 == 0 && (TA ? M % 4 == 0 : K % 4 == 0) && (TB ? K % 4 == 0 : true);
    const uint64_t tiles = (uint64_t)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
    if (tiles > 0x7fffffffull) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "sgemm: %u x %u too large", M, N);
    const bool valu = K > 0 && K <= kValuMaxK && (uint64_t)M * N * K <= kValuMaxWork;
    // Small grids (a K split of the 128 x 128 tiles, or the VALU split) on
    // the wave-split kernel when the operands suit its vector accesses
    // (RPLHIP_F32_WS=0 disables it, for A/B timing only).
    static const char* ws_env = getenv("RPLHIP_F32_WS");
    if (!valu && K > 0 && !(ws_env && ws_env[0] == '0') &&
        ((uint64_t)M * N * K <= kValuMaxWork || k_splits(tiles, K) > 1)) {
        const int st = wsk::launch<TA, TB>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c, bias, out2);
        if (st != -1) return st;
    }
    if (valu) {
        const uint64_t blocks = ((uint64_t)M * N + 255) / 256;  // M*N <= 2^23
        if constexpr (!TA && TB) {
            const size_t lds = valu_lds_bytes(N, K);
            if (lds && aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0) {
                hipLaunchKernelGGL(k_sgemm_valu_lds, dim3((uint32_t)blocks), dim3(256), lds, s, M, N, K, alpha, A, lda,
                                   B, ldb, beta, C, ldc, read_c, bias, out2);
                return rplhip::check_launch("sgemm (VALU, LDS)");
            }
            if (aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0) {
                hipLaunchKernelGGL((k_sgemm_valu<false, true, true>), dim3((uint32_t)blocks), dim3(256), 0, s, M, N,
                                   K, alpha, A, lda, B, ldb, beta, C, ldc, read_c, bias, out2);
                return rplhip::check_launch("sgemm (VALU)");
            }
        }
        hipLaunchKernelGGL((k_sgemm_valu<TA, TB, false>), dim3((uint32_t)blocks), dim3(256), 0, s, M, N, K, alpha, A,
                           lda, B, ldb, beta, C, ldc, read_c, bias, out2);
        return rplhip::check_launch("sgemm (VALU)");
    }
    if (K > kValuMaxK && (uint64_t)M * N * K <= kValuMaxWork) {
        uint32_t ns = (K + kValuSlice - 1) / kValuSlice;
        if (ns > kValuMaxSlices) ns = kValuMaxSlices;
        const uint32_t kps = (K + ns - 1) / ns;
        ns = (K + kps - 1) / kps;
        const uint32_t blocks = (uint32_t)(((uint64_t)M * N + 255) / 256);  // M*N <= 2^23 / 256
        void* ws = nullptr;
        int st = rplhip::ws_alloc(&ws, (size_t)ns * M * N * sizeof(float), s);
        if (st) return st;
        hipLaunchKernelGGL((k_sgemm_valu_split<TA, TB>), dim3(blocks, ns), dim3(256), 0, s, M, N, K, A, lda, B, ldb,
                           (float*)ws, kps);
        st = rplhip::check_launch("sgemm (VALU split-K)");
        if (!st) {
            hipLaunchKernelGGL(k_splitk_reduce, dim3(blocks), dim3(256), 0, s, (const float*)ws, ns, M, N, alpha, beta,
                               C, ldc, read_c, bias, out2);
            st = rplhip::check_launch("sgemm (VALU split-K reduction)");
        }
        rplhip::ws_free(ws, s);
        return st;
    }
    dim3 grid((uint32_t)tiles);
    // Big grids on the direct-to-LDS kernel (RPLHIP_F32_DMA=0 disables it,
    // for A/B timing only).
    static const char* dma_env = getenv("RPLHIP_F32_DMA");
    const uint64_t big_tiles = (uint64_t)((M + fd::BM - 1) / fd::BM) * ((N + fd::BN - 1) / fd::BN);
    const uint64_t a_bytes = (uint64_t)(TA ? K : M) * lda * 4, b_bytes = (uint64_t)(TB ? N : K) * ldb * 4;
    if (vec && K >= fd::BK && K % fd::BK == 0 && big_tiles >= 2ull * rplhip::cu_count() && a_bytes < (1ull << 31) &&
        b_bytes < (1ull << 31) && !(dma_env && dma_env[0] == '0')) {
        hipLaunchKernelGGL((k_sgemm_dma<TA, TB>), dim3((uint32_t)big_tiles), dim3(fd::kThreads), 0, s, M, N, K, alpha,
                           A, lda, B, ldb, beta, C, ldc, read_c);
        const int st = rplhip::check_launch("sgemm (direct-to-LDS)");
        return st || !bias ? st : rplhip_add_broadcast(C, bias, out2, (uint64_t)M * N, N, s);
    }
    const uint32_t splits = k_splits(tiles, K);
    if (splits > 1) {
        // Partial tiles into a stream-ordered workspace, then one reduction.
        uint32_t kps = (K + splits - 1) / splits;
        kps = (kps + BK - 1) / BK * BK;
        const uint32_t ns = (K + kps - 1) / kps;
        void* ws = nullptr;
        int st = rplhip::ws_alloc(&ws, (size_t)ns * M * N * sizeof(float), s);
        if (st) return st;
        dim3 g2(grid.x, ns);
        float* W = (float*)ws;
        if (vec)
            hipLaunchKernelGGL((k_sgemm<TA, TB, true, true>), g2, dim3(kThreads), 0, s, M, N, K, 1.0f, A, lda, B,
                               ldb, 0.0f, W, N, kps, 0ull, 0ull, 0ull, 1);
        else
            hipLaunchKernelGGL((k_sgemm<TA, TB, false, true>), g2, dim3(kThreads), 0, s, M, N, K, 1.0f, A, lda, B,
                               ldb, 0.0f, W, N, kps, 0ull, 0ull, 0ull, 1);
        st = rplhip::check_launch("sgemm (split-K)");
        if (!st) {
            const uint64_t total = (uint64_t)M * N;
            hipLaunchKernelGGL(k_splitk_reduce, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, W, ns, M, N,
                               alpha, beta, C, ldc, read_c, bias, out2);
            st = rplhip::check_launch("sgemm (split-K reduction)");
        }
        rplhip::ws_free(ws, s);
        return st;
    }
    if (vec)
        hipLaunchKernelGGL((k_sgemm<TA, TB, true, false>), grid, dim3(kThreads), 0, s, M, N, K, alpha, A, lda, B,
                           ldb, beta, C, ldc, K, 0ull, 0ull, 0ull, read_c);
    else
        hipLaunchKernelGGL((k_sgemm<TA, TB, false, false>), grid, dim3(kThreads), 0, s, M, N, K, alpha, A, lda, B,
                           ldb, beta, C, ldc, K, 0ull, 0ull, 0ull, read_c);
    const int st = rplhip::check_launch("sgemm");
    return st || !bias ? st : rplhip_add_broadcast(C, bias, out2, (uint64_t)M * N, N, s);
}

// `batch` GEMMs of one shape in one launch of the 128 x 128 kernel (grid z =
// batch index), C_z = alpha op(A_z) op(B_z) (+ beta C_z when read_c).
template <bool TA, bool TB>
int launch_batched(uint32_t M, uint32_t N, uint32_t K, float alpha, const float* A, uint32_t lda, uint64_t sA,
                   const float* B, uint32_t ldb, uint64_t sB, float beta, float* C, uint32_t ldc, uint64_t sC,
                   uint32_t batch, int read_c, hipStream_t s) {
    const bool vec = aligned16(A) && aligned16(B) && aligned16(C) && lda % 4 == 0 && ldb % 4 == 0 &&
                     ldc % 4 == 0 && N % 4 == 0 && (TA ? M % 4 == 0 : K % 4 == 0) && (TB ? K % 4 == 0 : true) &&
                     sA % 4 == 0 && sB % 4 == 0 && sC % 4 == 0;
    const uint64_t tiles = (uint64_t)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
    if (tiles > 0x7fffffffull) return rplhip::fail(RPLHIP_ERR_UNSUPPORTED, "sgemm: %u x %u too large", M, N);
    for (uint32_t b0 = 0; b0 < batch; b0 += 65535) {
        const uint32_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
        const dim3 grid((uint32_t)tiles, 1, nb);
        if (vec)
            hipLaunchKernelGGL((k_sgemm<TA, TB, true, false>), grid, dim3(kThreads), 0, s, M, N, K, alpha,
                               A + b0 * sA, lda, B + b0 * sB, ldb, beta, C + b0 * sC, ldc, K, sA, sB, sC, read_c);
        else
            hipLaunchKernelGGL((k_sgemm<TA, TB, false, false>), grid, dim3(kThreads), 0, s, M, N, K, alpha,
                               A + b0 * sA, lda, B + b0 * sB, ldb, beta, C + b0 * sC, ldc, K, sA, sB, sC, read_c);
        const int st = rplhip::check_launch("sgemm (batched)");
        if (st) return st;
    }
    return RPLHIP_OK;
}

}  // namespace

using namespace rplhip;

extern "C" int rplhip_sgemm(int trans_a, int trans_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                            const float* A, uint32_t lda, const float* B, uint32_t ldb, float beta, float* C,
                            uint32_t ldc, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!C || (K && (!A || !B))) return fail(RPLHIP_ERR_INVALID, "rplhip_sgemm: NULL pointer");
    if (ldc < N || (K && (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N))))
        return fail(RPLHIP_ERR_INVALID, "rplhip_sgemm: leading dimension too small");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (!trans_a && !trans_b) return launch<false, false>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (!trans_a && trans_b) return launch<false, true>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (trans_a && !trans_b) return launch<true, false>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    return launch<true, true>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
}

extern "C" int rplhip__linear_forward(const float* X, const float* W, const float* b, float* mm, float* out,
                                      uint32_t M, uint32_t N, uint32_t K, rplhip_stream_t stream) {
    if (M == 0 || N == 0) return RPLHIP_OK;
    if (!mm || !out || !b || (K && (!X || !W))) return fail(RPLHIP_ERR_INVALID, "rplhip__linear_forward: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    return launch<false, true>(M, N, K, 1.0f, X, K, W, K, 0.0f, mm, N, as_stream(stream), 0, b, out);
}

extern "C" int rplhip_sgemm_batched(int trans_a, int trans_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                                    const float* A, uint32_t lda, uint64_t stride_a, const float* B, uint32_t ldb,
                                    uint64_t stride_b, float beta, float* C, uint32_t ldc, uint64_t stride_c,
                                    uint32_t batch, int read_c, rplhip_stream_t stream) {
    if (M == 0 || N == 0 || batch == 0) return RPLHIP_OK;
    if (!C || (K && (!A || !B))) return fail(RPLHIP_ERR_INVALID, "rplhip_sgemm_batched: NULL pointer");
    if (ldc < N || (K && (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N))))
        return fail(RPLHIP_ERR_INVALID, "rplhip_sgemm_batched: leading dimension too small");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (batch == 1) {  // one product: the full dispatch (large tiles, split-K)
        if (!trans_a && !trans_b) return launch<false, false>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c);
        if (!trans_a && trans_b) return launch<false, true>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c);
        if (trans_a && !trans_b) return launch<true, false>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c);
        return launch<true, true>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s, read_c);
    }
    if (!trans_a && !trans_b)
        return launch_batched<false, false>(M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                                            stride_c, batch, read_c, s);
    if (!trans_a && trans_b)
        return launch_batched<false, true>(M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                                           stride_c, batch, read_c, s);
    if (trans_a && !trans_b)
        return launch_batched<true, false>(M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                                           stride_c, batch, read_c, s);
    return launch_batched<true, true>(M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc, stride_c,
                                      batch, read_c, s);
}
