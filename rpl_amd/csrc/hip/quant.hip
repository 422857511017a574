// Quantize / dequantize / min-max kernels (bit-exact with the reference).
//
// All of these are HBM-bound streaming passes: 128-bit loads and stores,
// grid-stride loops sized to fill the 256 CUs, and deterministic two-stage
// reductions (per-block partials in a stream-ordered workspace, then one
// finishing block) instead of float atomics.
#include <float.h>
#include <math.h>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 1024;

__device__ __forceinline__ float sel_min(float v, float m) { return v < m ? v : m; }
__device__ __forceinline__ float sel_max(float v, float m) { return v > m ? v : m; }

// Block-wide reduction of (min, max) with NaN never selected; every thread
// gets the result.
__device__ void block_min_max(float& mn, float& mx) {
    __shared__ float smin[kThreads / 64], smax[kThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        mn = sel_min(__shfl_xor(mn, off), mn);
        mx = sel_max(__shfl_xor(mx, off), mx);
    }
    int w = threadIdx.x / 64, l = threadIdx.x % 64;
    if (l == 0) { smin[w] = mn; smax[w] = mx; }
    __syncthreads();
    mn = smin[0];
    mx = smax[0];
    for (int i = 1; i < (int)(blockDim.x / 64); i++) {
        mn = sel_min(smin[i], mn);
        mx = sel_max(smax[i], mx);
    }
    __syncthreads();
}

// Stage 1: per-block (min, max) of x[0..n), OpenMP-reduction semantics.
__global__ void __launch_bounds__(kThreads) k_min_max_partial(const float* __restrict__ x, uint64_t n,
                                                              float2* __restrict__ part) {
    float mn = FLT_MAX, mx = -FLT_MAX;
    uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    bool vec = (((uintptr_t)x) & 15) == 0;
    if (vec) {
        uint64_t n4 = n / 4;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        for (uint64_t i = tid; i < n4; i += stride) {
            float4 v = x4[i];
            mn = sel_min(v.x, mn); mx = sel_max(v.x, mx);
            mn = sel_min(v.y, mn); mx = sel_max(v.y, mx);
            mn = sel_min(v.z, mn); mx = sel_max(v.z, mx);
            mn = sel_min(v.w, mn); mx = sel_max(v.w, mx);
        }
        for (uint64_t i = n4 * 4 + tid; i < n; i += stride) {
            mn = sel_min(x[i], mn);
            mx = sel_max(x[i], mx);
        }
    } else {
        for (uint64_t i = tid; i < n; i += stride) {
            mn = sel_min(x[i], mn);
            mx = sel_max(x[i], mx);
        }
    }
    block_min_max(mn, mx);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(mn, mx);
}

// Which parameters the finishing block derives from the global (min, max).
enum Finish { kMinMax = 0, kSymmetric = 1, kAsymmetric = 2 };

// Stage 2 (one block): combine partials and derive the quantization params.
//   kMinMax:     out2 = {min, max}
//   kSymmetric:  scale = fmaxf(fabsf(min), fabsf(max)) / 127  (rpl_quantization.c:87-88)
//   kAsymmetric: scale = (max - min) / 255, zp = (int32)roundf(-min / scale)  (:102-104)
template <int F>
__global__ void __launch_bounds__(kThreads) k_min_max_finish(const float2* __restrict__ part, int nparts,
                                                             float* __restrict__ out_f,
                                                             int32_t* __restrict__ out_zp) {
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
        float2 p = part[i];
        mn = sel_min(p.x, mn);
        mx = sel_max(p.y, mx);
    }
    block_min_max(mn, mx);
    if (threadIdx.x != 0) return;
    if (F == kMinMax) {
        out_f[0] = mn;
        out_f[1] = mx;
    } else if (F == kSymmetric) {
        float abs_max = fmaxf(fabsf(mn), fabsf(mx));
        out_f[0] = abs_max / 127.0f;
    } else {
        float range = mx - mn;
        float scale = range / 255.0f;
        out_f[0] = scale;
        out_zp[0] = x86_cvt_i32(roundf(-mn / scale));
    }
}

// q = quantize_one(x, scale, zp); scale / zp come from device memory when
// the pointers are given (symmetric / asymmetric chains), else the values.
__global__ void __launch_bounds__(kThreads) k_quantize(const float* __restrict__ x, uint64_t n,
                                                       float scale_v, int32_t zp_v,
                                                       const float* __restrict__ scale_p,
                                                       const int32_t* __restrict__ zp_p,
                                                       int8_t* __restrict__ q) {
    float scale = scale_p ? *scale_p : scale_v;
    int32_t zp = zp_p ? *zp_p : zp_v;
    uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    bool vec = ((((uintptr_t)x) & 15) == 0) && ((((uintptr_t)q) & 3) == 0);
    uint64_t n4 = vec ? n / 4 : 0;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    uint32_t* q4 = reinterpret_cast<uint32_t*>(q);
    for (uint64_t i = tid; i < n4; i += stride) {
        float4 v = x4[i];
        uint32_t b0 = (uint8_t)quantize_one(v.x, scale, zp);
        uint32_t b1 = (uint8_t)quantize_one(v.y, scale, zp);
        uint32_t b2 = (uint8_t)quantize_one(v.z, scale, zp);
        uint32_t b3 = (uint8_t)quantize_one(v.w, scale, zp);
        q4[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    for (uint64_t i = n4 * 4 + tid; i < n; i += stride) q[i] = quantize_one(x[i], scale, zp);
}

// Stage 2 and the quantization in one launch: every block combines the
// (few) stage-1 partials itself, derives the parameters exactly as
// k_min_max_finish<F> does (min / max selection is order-free, the formulas
// are the same), block 0 stores them, and the block quantizes its share of
// x as k_quantize does.
template <int F>
__global__ void __launch_bounds__(kThreads) k_quantize_chain(const float* __restrict__ x, uint64_t n,
                                                             const float2* __restrict__ part, int nparts,
                                                             float* __restrict__ out_f, int32_t* __restrict__ out_zp,
                                                             int8_t* __restrict__ q) {
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
        float2 p = part[i];
        mn = sel_min(p.x, mn);
        mx = sel_max(p.y, mx);
    }
    block_min_max(mn, mx);
    float scale;
    int32_t zp = 0;
    if (F == kSymmetric) {
        scale = fmaxf(fabsf(mn), fabsf(mx)) / 127.0f;
    } else {
        const float range = mx - mn;
        scale = range / 255.0f;
        zp = x86_cvt_i32(roundf(-mn / scale));
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        out_f[0] = scale;
        if (F == kAsymmetric) out_zp[0] = zp;
    }
    uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    bool vec = ((((uintptr_t)x) & 15) == 0) && ((((uintptr_t)q) & 3) == 0);
    uint64_t n4 = vec ? n / 4 : 0;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    uint32_t* q4 = reinterpret_cast<uint32_t*>(q);
    for (uint64_t i = tid; i < n4; i += stride) {
        float4 v = x4[i];
        uint32_t b0 = (uint8_t)quantize_one(v.x, scale, zp);
        uint32_t b1 = (uint8_t)quantize_one(v.y, scale, zp);
        uint32_t b2 = (uint8_t)quantize_one(v.z, scale, zp);
        uint32_t b3 = (uint8_t)quantize_one(v.w, scale, zp);
        q4[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    for (uint64_t i = n4 * 4 + tid; i < n; i += stride) q[i] = quantize_one(x[i], scale, zp);
}

// y = (float)(q - zp) * scale  (ops_extended.c:69)
__global__ void __launch_bounds__(kThreads) k_dequantize(const int8_t* __restrict__ q, uint64_t n,
                                                         float scale, int32_t zp,
                                                         float* __restrict__ y) {
    uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    bool vec = ((((uintptr_t)q) & 3) == 0) && ((((uintptr_t)y) & 15) == 0);
    uint64_t n4 = vec ? n / 4 : 0;
    const uint32_t* q4 = reinterpret_cast<const uint32_t*>(q);
    float4* y4 = reinterpret_cast<float4*>(y);
    for (uint64_t i = tid; i < n4; i += stride) {
        uint32_t w = q4[i];
        float4 o;
        o.x = (float)((int32_t)(int8_t)(w & 0xff) - zp) * scale;
        o.y = (float)((int32_t)(int8_t)((w >> 8) & 0xff) - zp) * scale;
        o.z = (float)((int32_t)(int8_t)((w >> 16) & 0xff) - zp) * scale;
        o.w = (float)((int32_t)(int8_t)(w >> 24) - zp) * scale;
        y4[i] = o;
    }
    for (uint64_t i = n4 * 4 + tid; i < n; i += stride) y[i] = (float)((int32_t)q[i] - zp) * scale;
}

// Per-channel (per-row) symmetric quantization: min/max over the slice,
// scale = fmaxf(|min|,|max|)/127, then quantize (src/rpl_quantization.c:
// 120-160).  The reference scans with `x < min` / `x > max` from FLT_MAX /
// -FLT_MAX, so NaN is never taken and fmaxf(|min|,|max|) is the largest |x|
// over the slice's non-NaN elements, or FLT_MAX when it has none; the
// kernels compute that directly, in any order.
//
// Division by a row's scale s: when 2^-100 <= s <= 2^125, q = x * inv with
// inv = 1.0f / s correctly rounded, then one FMA correction
// q' = fma(fma(-q, s, x), inv, q).  For |x| >= s/4 the residual x - q*s is
// a multiple of 2^-148, hence exact, and q' is x / s correctly rounded
// (Markstein's theorem: inv within half an ulp of 1/s, q within an ulp of
// x/s); below s/4 q' may differ from x / s in its last bits, but both are
// below 1/2 in magnitude and quantize to 0.  3 VALU operations instead of
// the ~10 of a general IEEE divide.  Other scales (0 for an all-zero slice,
// inf, tiny or huge) divide exactly.  Checked against x / s on the CPU
// (tests/quant_div_identity.c).
__device__ __forceinline__ float div_scale_fast(float x, float s, float inv) {
#pragma clang fp contract(off)
    const float q = x * inv;
    return __builtin_fmaf(__builtin_fmaf(-q, s, x), inv, q);
}
__device__ __forceinline__ bool scale_fast_ok(float s) { return s >= 0x1p-100f && s <= 0x1p125f; }

// clamp(x86((int32)roundf(y)), -128, 127) as a byte.
__device__ __forceinline__ uint32_t q8_of(float y) {
    const int32_t v = x86_round_cvt(y);
    return (uint8_t)(int8_t)(v < -128 ? -128 : (v > 127 ? 127 : v));
}
// The same for |y| < 2^31 or NaN (the quotients of the fast division are
// at most 128 in magnitude): roundf(y) = trunc(y + copysign(0.49999997, y)),
// clamped before the truncating conversion; fmaxf takes -128 for a NaN,
// which is where x86's INT32_MIN clamps.  5 VALU operations.
__device__ __forceinline__ uint32_t q8_small(float y) {
#pragma clang fp contract(off)
    const float t = y + __builtin_copysignf(0.49999997f, y);
    return (uint32_t)(int32_t)__builtin_fminf(__builtin_fmaxf(t, -128.0f), 127.0f);
}
// Low bytes of four words packed into one (v_perm_b32).
__device__ __forceinline__ uint32_t pack4(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u) | __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);
}

// k_quantize_rows_wave: WPR waves per slice of up to 256*NV*WPR floats
// (cols % 4 == 0, 16-byte aligned rows), 4/WPR slices per block.  Lane l of
// the slice's 64*WPR lanes holds float4 items l, l + 64 WPR, .. in
// registers, so the slice is read from HBM once; every load is unconditional
// (items past the slice re-read its last float4, which leaves the largest
// |x| unchanged) so all NV loads are in flight together.  The reduction is
// wave-local, then across the slice's waves through LDS when WPR > 1.  FULL:
// the slice is exactly 256*NV*WPR floats.  NT: non-temporal loads (X is read
// once).  Measured on 2048 x 4096 (config 3's tokens): one wave per row,
// 11.5 us with X in HBM (6.7 us from the MALL); 4 waves per row with NT
// loads, 8.5 us (6.6 us); 2 or 8 waves, or NT loads with one wave, in between.
template <int NV, int WPR, bool FULL, bool NT>
__global__ void __launch_bounds__(kThreads) k_quantize_rows_wave(const float* __restrict__ x, uint32_t rows,
                                                                 uint32_t cols, int8_t* __restrict__ q,
                                                                 float* __restrict__ scales) {
    static_assert(kThreads == 256 && 4 % WPR == 0, "4 waves per block, WPR of them per slice");
    constexpr uint32_t T = 64 * WPR;
    const uint32_t r = blockIdx.x * (4 / WPR) + threadIdx.x / T;
    // With WPR == 1 a wave past the last slice leaves at once; with WPR > 1
    // the grid has exactly one block per slice group (rows % (4 / WPR) is
    // handled by `live`), so every wave reaches the barrier.
    const bool live = r < rows;
    if (WPR == 1 && !live) return;
    const uint32_t lane = threadIdx.x % T, n4 = cols / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x + (uint64_t)(live ? r : 0) * cols);
    float4 v[NV];
#pragma unroll
    for (int it = 0; it < NV; it++) {
        const uint32_t i = lane + T * it;
        const float4* p = x4 + (FULL || i < n4 ? i : n4 - 1);
        if (NT) {
            const v4f t = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
            v[it] = make_float4(t[0], t[1], t[2], t[3]);
        } else {
            v[it] = *p;
        }
    }
    // Largest |x| over non-NaN elements (fmaxf returns the other operand
    // for a NaN); -1 when there is none.
    float amax = -1.0f;
#pragma unroll
    for (int it = 0; it < NV; it++) {
        amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fabsf(v[it].x), __builtin_fabsf(v[it].y)));
        amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fabsf(v[it].z), __builtin_fabsf(v[it].w)));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = __builtin_fmaxf(__shfl_xor(amax, off), amax);
    if constexpr (WPR > 1) {
        __shared__ float red[4];
        const uint32_t w = threadIdx.x / 64;
        if (threadIdx.x % 64 == 0) red[w] = amax;
        __syncthreads();
        const uint32_t w0 = w / WPR * WPR;
        amax = red[w0];
#pragma unroll
        for (int i = 1; i < WPR; i++) amax = __builtin_fmaxf(amax, red[w0 + i]);
        if (!live) return;
    }
    const float scale = (amax < 0.0f ? FLT_MAX : amax) / 127.0f;
    if (lane == 0) scales[r] = scale;
    uint32_t* q4 = reinterpret_cast<uint32_t*>(q + (uint64_t)r * cols);
    const bool fast = scale_fast_ok(scale);  // uniform over the slice
    const float inv = 1.0f / scale;
#pragma unroll
    for (int it = 0; it < NV; it++) {
        const uint32_t i = lane + T * it;
        if (FULL || i < n4) {
            const float4 t = v[it];
            uint32_t w;
            if (fast)
                w = pack4(q8_small(div_scale_fast(t.x, scale, inv)), q8_small(div_scale_fast(t.y, scale, inv)),
                          q8_small(div_scale_fast(t.z, scale, inv)), q8_small(div_scale_fast(t.w, scale, inv)));
            else
                w = pack4(q8_of(t.x / scale), q8_of(t.y / scale), q8_of(t.z / scale), q8_of(t.w / scale));
            q4[i] = w;
        }
    }
}
constexpr uint32_t kRowsWaveMaxCols = 256 * 32;

// Other slices (cols % 4 != 0, unaligned rows, or more than
// kRowsWaveMaxCols floats): one block per slice, read twice.
__global__ void __launch_bounds__(kThreads) k_quantize_rows(const float* __restrict__ x, uint32_t rows,
                                                            uint32_t cols, int8_t* __restrict__ q,
                                                            float* __restrict__ scales) {
    uint32_t r = blockIdx.x;
    const float* xr = x + (uint64_t)r * cols;
    int8_t* qr = q + (uint64_t)r * cols;
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (uint32_t i = threadIdx.x; i < cols; i += kThreads) {
        mn = sel_min(xr[i], mn);
        mx = sel_max(xr[i], mx);
    }
    block_min_max(mn, mx);
    float scale = fmaxf(fabsf(mn), fabsf(mx)) / 127.0f;
    if (threadIdx.x == 0) scales[r] = scale;
    for (uint32_t i = threadIdx.x; i < cols; i += kThreads) qr[i] = quantize_one(xr[i], scale, 0);
}

// tensor_get_min_max: first index attaining the extreme wins.
struct ArgExt {
    float mn;
    uint64_t imn;
    float mx;
    uint64_t imx;
};

__device__ __forceinline__ void argext_merge(ArgExt& a, float vmn, uint64_t imn, float vmx,
                                             uint64_t imx) {
    if (vmn < a.mn || (vmn == a.mn && imn < a.imn)) { a.mn = vmn; a.imn = imn; }
    if (vmx > a.mx || (vmx == a.mx && imx < a.imx)) { a.mx = vmx; a.imx = imx; }
}

__device__ void block_argext(ArgExt& a) {
    __shared__ ArgExt s[kThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        float vmn = __shfl_xor(a.mn, off);
        uint64_t imn = __shfl_xor(a.imn, off);
        float vmx = __shfl_xor(a.mx, off);
        uint64_t imx = __shfl_xor(a.imx, off);
        argext_merge(a, vmn, imn, vmx, imx);
    }
    int w = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) s[w] = a;
    __syncthreads();
    a = s[0];
    for (int i = 1; i < (int)(blockDim.x / 64); i++) argext_merge(a, s[i].mn, s[i].imn, s[i].mx, s[i].imx);
    __syncthreads();
}

__global__ void __launch_bounds__(kThreads) k_argext_partial(const float* __restrict__ x, uint64_t n,
                                                             ArgExt* __restrict__ part) {
    ArgExt a = {__builtin_huge_valf(), ~0ull, -__builtin_huge_valf(), ~0ull};
    uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = tid; i < n; i += stride) {
        float v = x[i];
        if (v == v) argext_merge(a, v, i, v, i);  // NaN never selected past x[0]
    }
    block_argext(a);
    if (threadIdx.x == 0) part[blockIdx.x] = a;
}

__global__ void __launch_bounds__(kThreads) k_argext_finish(const float* __restrict__ x,
                                                            const ArgExt* __restrict__ part,
                                                            int nparts, float* __restrict__ out2) {
    ArgExt a = {__builtin_huge_valf(), ~0ull, -__builtin_huge_valf(), ~0ull};
    for (int i = threadIdx.x; i < nparts; i += blockDim.x)
        argext_merge(a, part[i].mn, part[i].imn, part[i].mx, part[i].imx);
    block_argext(a);
    if (threadIdx.x != 0) return;
    float x0 = x[0];
    if (x0 != x0) {  // the scan starts from x[0]; a NaN there is never replaced
        out2[0] = x0;
        out2[1] = x0;
        return;
    }
    // All elements are compared against x[0] first, so a non-NaN x[0] is a
    // candidate; the merged arg-extremes already include it (index 0).
    out2[0] = x[a.imn];
    out2[1] = x[a.imx];
}

int grid_for(uint64_t work_items) {
    uint64_t b = (work_items + kThreads - 1) / kThreads;
    if (b < 1) b = 1;
    int cap = kMaxBlocks;
    return (int)(b < (uint64_t)cap ? b : (uint64_t)cap);
}

// Shared two-stage min/max with a finishing mode.
template <int F>
int min_max_chain(const float* x, uint64_t n, float* out_f, int32_t* out_zp, hipStream_t s) {
    int g = grid_for((n + 3) / 4);
    void* ws = nullptr;
    int st = rplhip::ws_alloc(&ws, sizeof(float2) * g, s);
    if (st) return st;
    hipLaunchKernelGGL(k_min_max_partial, dim3(g), dim3(kThreads), 0, s, x, n, (float2*)ws);
    hipLaunchKernelGGL(k_min_max_finish<F>, dim3(1), dim3(kThreads), 0, s, (const float2*)ws, g,
                       out_f, out_zp);
    st = rplhip::check_launch("min/max reduction");
    rplhip::ws_free(ws, s);
    return st;
}

// Symmetric / asymmetric quantization of x[0..n), n > 0: min/max partials,
// then k_quantize_chain (two launches).
template <int F>
int quantize_chain(const float* x, uint64_t n, int8_t* q, float* out_f, int32_t* out_zp, hipStream_t s) {
    int g = grid_for((n + 3) / 4);
    void* ws = nullptr;
    int st = rplhip::ws_alloc(&ws, sizeof(float2) * g, s);
    if (st) return st;
    hipLaunchKernelGGL(k_min_max_partial, dim3(g), dim3(kThreads), 0, s, x, n, (float2*)ws);
    hipLaunchKernelGGL(k_quantize_chain<F>, dim3(g), dim3(kThreads), 0, s, x, n, (const float2*)ws, g, out_f,
                       out_zp, q);
    st = rplhip::check_launch("quantize");
    rplhip::ws_free(ws, s);
    return st;
}

}  // namespace

using namespace rplhip;

extern "C" {

int rplhip_quantize_int8(const float* x, uint64_t n, float scale, int32_t zp, int8_t* q,
                         rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !q) return fail(RPLHIP_ERR_INVALID, "rplhip_quantize_int8: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(k_quantize, dim3(grid_for((n + 3) / 4)), dim3(kThreads), 0, s, x, n, scale, zp,
                       (const float*)nullptr, (const int32_t*)nullptr, q);
    return check_launch("quantize_int8");
}

int rplhip_min_max(const float* x, uint64_t n, float* out2, rplhip_stream_t stream) {
    if (!x || !out2) return fail(RPLHIP_ERR_INVALID, "rplhip_min_max: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    return min_max_chain<kMinMax>(x, n, out2, nullptr, as_stream(stream));
}

int rplhip_quantize_symmetric(const float* x, uint64_t n, int8_t* q, float* scale_out,
                              rplhip_stream_t stream) {
    if (!x || !q || !scale_out) return fail(RPLHIP_ERR_INVALID, "rplhip_quantize_symmetric: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (n == 0) return min_max_chain<kSymmetric>(x, n, scale_out, nullptr, s);
    return quantize_chain<kSymmetric>(x, n, q, scale_out, nullptr, s);
}

int rplhip_quantize_asymmetric(const float* x, uint64_t n, int8_t* q, float* scale_out,
                               int32_t* zp_out, rplhip_stream_t stream) {
    if (!x || !q || !scale_out || !zp_out)
        return fail(RPLHIP_ERR_INVALID, "rplhip_quantize_asymmetric: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (n == 0) return min_max_chain<kAsymmetric>(x, n, scale_out, zp_out, s);
    return quantize_chain<kAsymmetric>(x, n, q, scale_out, zp_out, s);
}

int rplhip_quantize_per_channel(const float* x, uint32_t num_channels, uint32_t channel_size,
                                int8_t* q, float* scales, rplhip_stream_t stream) {
    if (num_channels == 0) return RPLHIP_OK;
    if (!x || !q || !scales) return fail(RPLHIP_ERR_INVALID, "rplhip_quantize_per_channel: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    const bool reg = channel_size > 0 && channel_size % 4 == 0 && channel_size <= kRowsWaveMaxCols && (((uintptr_t)x) & 15) == 0 &&
                     (((uintptr_t)q) & 3) == 0;
    if (reg && channel_size >= 1024) {
        // 4 waves per slice, one slice per block, non-temporal loads
        const dim3 grid(num_channels);
        const uint32_t nv = (channel_size + 1023) / 1024;
#define RPL_QR(NV)                                                                                            \
    do {                                                                                                      \
        if (channel_size == 1024 * NV)                                                                        \
            hipLaunchKernelGGL((k_quantize_rows_wave<NV, 4, true, true>), grid, dim3(kThreads), 0, s, x,       \
                               num_channels, channel_size, q, scales);                                        \
        else                                                                                                  \
            hipLaunchKernelGGL((k_quantize_rows_wave<NV, 4, false, true>), grid, dim3(kThreads), 0, s, x,      \
                               num_channels, channel_size, q, scales);                                        \
    } while (0)
        if (nv <= 1)
            RPL_QR(1);
        else if (nv <= 2)
            RPL_QR(2);
        else if (nv <= 4)
            RPL_QR(4);
        else
            RPL_QR(8);
#undef RPL_QR
    } else if (reg) {
        // shorter slices: one wave each
        const dim3 grid((num_channels + kThreads / 64 - 1) / (kThreads / 64));
        const uint32_t nv = (channel_size + 255) / 256;
#define RPL_QR(NV)                                                                                         \
    do {                                                                                                   \
        if (channel_size == 256 * NV)                                                                      \
            hipLaunchKernelGGL((k_quantize_rows_wave<NV, 1, true, false>), grid, dim3(kThreads), 0, s, x,   \
                               num_channels, channel_size, q, scales);                                     \
        else                                                                                               \
            hipLaunchKernelGGL((k_quantize_rows_wave<NV, 1, false, false>), grid, dim3(kThreads), 0, s, x,  \
                               num_channels, channel_size, q, scales);                                     \
    } while (0)
        if (nv <= 1)
            RPL_QR(1);
        else if (nv <= 2)
            RPL_QR(2);
        else
            RPL_QR(4);
#undef RPL_QR
    } else {
        hipLaunchKernelGGL(k_quantize_rows, dim3(num_channels), dim3(kThreads), 0, s, x, num_channels, channel_size,
                           q, scales);
    }
    return check_launch("quantize_per_channel");
}

int rplhip_dequantize_int8(const int8_t* q, uint64_t n, float scale, int32_t zp, float* y,
                           rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!q || !y) return fail(RPLHIP_ERR_INVALID, "rplhip_dequantize_int8: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_dequantize, dim3(grid_for((n + 3) / 4)), dim3(kThreads), 0, as_stream(stream),
                       q, n, scale, zp, y);
    return check_launch("dequantize_int8");
}

int rplhip_get_min_max(const float* x, uint64_t n, float* out2, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !out2) return fail(RPLHIP_ERR_INVALID, "rplhip_get_min_max: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    int g = grid_for(n);
    void* ws = nullptr;
    int st = ws_alloc(&ws, sizeof(ArgExt) * g, s);
    if (st) return st;
    hipLaunchKernelGGL(k_argext_partial, dim3(g), dim3(kThreads), 0, s, x, n, (ArgExt*)ws);
    hipLaunchKernelGGL(k_argext_finish, dim3(1), dim3(kThreads), 0, s, x, (const ArgExt*)ws, g, out2);
    st = check_launch("get_min_max");
    ws_free(ws, s);
    return st;
}

}  // extern "C"
