// Elementwise and reduction kernels around the Linear GEMMs: bias add (+ReLU),
// ReLU backward, gradient accumulation, the bias-gradient column reduction and
// the MSE loss / backward.  All are HBM- or launch-bound; the GEMMs dominate.
#include <math.h>

#include "common.h"
#include "rplhip_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 2048;

int grid_for(uint64_t items) {
    uint64_t b = (items + kThreads - 1) / kThreads;
    if (b < 1) b = 1;
    return (int)(b < (uint64_t)kMaxBlocks ? b : (uint64_t)kMaxBlocks);
}

#define GRID_STRIDE(i, n)                                                          \
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); \
         i += (uint64_t)gridDim.x * blockDim.x)

// out[i] = a[i] + b[i % nb]; act[i] = relu(out[i]) when act != NULL
// (rpl_core.c:112-120 then :291).
__global__ void __launch_bounds__(kThreads) k_bias_add_relu(const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            float* __restrict__ out,
                                                            float* __restrict__ act, uint64_t n,
                                                            uint64_t nb) {
    GRID_STRIDE(i, n) {
        float v = a[i] + b[i % nb];
        out[i] = v;
        if (act) act[i] = v > 0 ? v : 0;
    }
}

__global__ void __launch_bounds__(kThreads) k_relu(const float* __restrict__ x, float* __restrict__ y,
                                                   uint64_t n) {
    GRID_STRIDE(i, n) {
        float v = x[i];
        y[i] = v > 0 ? v : 0;
    }
}

// rpl_core.c:421: the new value of one element of the input's gradient.
// overwrite: the gradient holds zeros only logically (0.0f + dy, or 0.0f
// where x <= 0: the bits of the accumulation into +0.0); else base += dy
// where x > 0.
__device__ __forceinline__ float relu_grad_acc(bool overwrite, float base, float x, float dy) {
    return overwrite ? (x > 0 ? 0.0f + dy : 0.0f) : (x > 0 ? base + dy : base);
}
__global__ void __launch_bounds__(kThreads) k_relu_backward(const float* __restrict__ x,
                                                            const float* __restrict__ dy,
                                                            float* __restrict__ dx, uint64_t n, int overwrite) {
    if (overwrite) {
        GRID_STRIDE(i, n) { dx[i] = relu_grad_acc(true, 0.0f, x[i], dy[i]); }
    } else {
        GRID_STRIDE(i, n) {
            if (x[i] > 0) dx[i] = relu_grad_acc(false, dx[i], x[i], dy[i]);
        }
    }
}

// rpl_core.c:441-444: one element of the predictions' gradient, base +
// (g0 * 2/n) * (p - t), which contracts to fma(g0f, p - t, base).
__device__ __forceinline__ float mse_grad_acc(float base, float g0f, float p, float t) { return base + g0f * (p - t); }

// rpl_core.c:324 (overwrite: dx = 0.0f + dy, as into a zeroed dx)
__global__ void __launch_bounds__(kThreads) k_accumulate(const float* __restrict__ dy,
                                                         float* __restrict__ dx, uint64_t n, int overwrite) {
    GRID_STRIDE(i, n) { dx[i] = (overwrite ? 0.0f : dx[i]) + dy[i]; }
}

__global__ void __launch_bounds__(kThreads) k_fill(float* __restrict__ x, uint64_t n, float v) {
    GRID_STRIDE(i, n) { x[i] = v; }
}

// Bias-gradient column reduction, stage 1: dy viewed as [rows, nb]; block
// (cx, split) sums 64 columns over its slice of rows with 4 row lanes, so
// each wave reads 64 consecutive floats of a row (coalesced).
constexpr int kColTile = 64;
constexpr int kRowLanes = kThreads / kColTile;

// DX: also pass the gradient through to backward_add's other operand,
// dx = dx + dy (overwrite: 0.0f + dy), as k_accumulate does; every element
// of dy is visited exactly once.
// SRC: where dy comes from.  kSrcGrad: read it.  kSrcRelu / kSrcMse: it is
// the add output's gradient right after the ReLU / MSE backward that
// follows the add in the graph accumulated into it (the autograd walk runs
// backward_add right after that accumulation): the element is computed
// here as k_relu_backward / k_mse_backward would, written to that gradient,
// and used as dy (one pass instead of two).
enum { kSrcGrad = 0, kSrcRelu = 1, kSrcMse = 2 };
template <bool DX, int SRC>
__global__ void __launch_bounds__(kThreads) k_colsum_partial(const float* __restrict__ dy, uint64_t n,
                                                             uint64_t rows, uint64_t nb,
                                                             uint64_t rows_per_split,
                                                             float* __restrict__ part, float* __restrict__ dx,
                                                             int dx_overwrite, RplGradSrc src) {
    __shared__ float red[kRowLanes][kColTile];
    uint64_t c = (uint64_t)blockIdx.x * kColTile + threadIdx.x % kColTile;
    int lane_r = threadIdx.x / kColTile;
    uint64_t r0 = (uint64_t)blockIdx.y * rows_per_split;
    uint64_t r1 = r0 + rows_per_split < rows ? r0 + rows_per_split : rows;
    const float g0f = SRC == kSrcMse ? (src.g0p ? *src.g0p : src.g0v) * (2.0f / (float)n) : 0.0f;
    // dy at element i (SRC != kSrcGrad: also written to the add output's
    // gradient).
    auto value = [&](uint64_t i) {
        if constexpr (SRC == kSrcGrad) {
            return dy[i];
        } else {
            const float base = src.g_overwrite ? 0.0f : src.g[i];
            const float v = SRC == kSrcRelu ? relu_grad_acc(src.g_overwrite, base, src.x[i], src.y[i])
                                            : mse_grad_acc(base, g0f, src.x[i], src.y[i]);
            src.g[i] = v;
            return v;
        }
    };
    // Rows in batches of 4 loads in flight, added in row order (a chain of
    // one load per row was latency-bound: 6-7 us for [4096, 128]).
    float g = 0;
    if (c < nb) {
        uint64_t r = r0 + lane_r;
        for (; r + 3 * kRowLanes < r1; r += 4 * kRowLanes) {
            float v[4];
            bool ok[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint64_t i = (r + j * kRowLanes) * nb + c;
                ok[j] = i < n;
                v[j] = ok[j] ? value(i) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (ok[j]) g += v[j];
            if constexpr (DX) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint64_t i = (r + j * kRowLanes) * nb + c;
                    if (ok[j]) dx[i] = (dx_overwrite ? 0.0f : dx[i]) + v[j];
                }
            }
        }
        for (; r < r1; r += kRowLanes)
            if (r * nb + c < n) {
                const float v = value(r * nb + c);
                g += v;
                if constexpr (DX) dx[r * nb + c] = (dx_overwrite ? 0.0f : dx[r * nb + c]) + v;
            }
    }
    red[lane_r][threadIdx.x % kColTile] = g;
    __syncthreads();
    if (lane_r == 0 && c < nb) {
        float s = red[0][threadIdx.x];
        for (int k = 1; k < kRowLanes; k++) s += red[k][threadIdx.x];
        part[(uint64_t)blockIdx.y * nb + c] = s;
    }
}
// Stage 2: db[c] (+)= the sum of column c's split partials.  A block takes
// 16 columns with 16 lanes each; lane l adds partials l, l+16, .. (4 loads in
// flight), then lane 0 adds the 16 lane sums in lane order.
constexpr int kFinCols = 16, kFinLanes = kThreads / kFinCols;
__global__ void __launch_bounds__(kThreads) k_colsum_finish(const float* __restrict__ part, int splits,
                                                            uint64_t nb, float* __restrict__ db, int overwrite) {
    __shared__ float red[kFinLanes][kFinCols];
    const uint64_t c = (uint64_t)blockIdx.x * kFinCols + threadIdx.x % kFinCols;
    const int lane = threadIdx.x / kFinCols;
    float s = 0;
    if (c < nb) {
        int k = lane;
        for (; k + 3 * kFinLanes < splits; k += 4 * kFinLanes) {
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = part[(uint64_t)(k + j * kFinLanes) * nb + c];
#pragma unroll
            for (int j = 0; j < 4; j++) s += v[j];
        }
        for (; k < splits; k += kFinLanes) s += part[(uint64_t)k * nb + c];
    }
    red[lane][threadIdx.x % kFinCols] = s;
    __syncthreads();
    if (lane == 0 && c < nb) {
        float t = red[0][threadIdx.x];
        for (int r = 1; r < kFinLanes; r++) t += red[r][threadIdx.x];
        db[c] = (overwrite ? 0.0f : db[c]) + t;
    }
}

// MSE: per-block partial sums of (p - t)^2, then one block finishes.
__device__ float block_sum(float v) {
    __shared__ float s[kThreads / 64];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (threadIdx.x % 64 == 0) s[threadIdx.x / 64] = v;
    __syncthreads();
    float t = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); i++) t += s[i];
    __syncthreads();
    return t;
}

__global__ void __launch_bounds__(kThreads) k_sqerr_partial(const float* __restrict__ p,
                                                            const float* __restrict__ t, uint64_t n,
                                                            float* __restrict__ part) {
    float acc = 0;
    GRID_STRIDE(i, n) {
        float d = p[i] - t[i];
        acc += d * d;
    }
    acc = block_sum(acc);
    if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

__global__ void __launch_bounds__(kThreads) k_sqerr_finish(const float* __restrict__ part, int nparts,
                                                           uint64_t n, float* __restrict__ loss) {
    float acc = 0;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) acc += part[i];
    acc = block_sum(acc);
    if (threadIdx.x == 0) loss[0] = acc / (float)n;  // rpl_core.c:457
}

// n <= kSqerrSingleMax: the whole sum in one block (one launch instead of
// partials plus a finishing block): a strided sum per thread (4 consecutive
// elements per step when aligned), a 64-lane butterfly, then the 16 wave sums
// in order.
constexpr int kSqerrThreads = 1024;
constexpr uint64_t kSqerrSingleMax = uint64_t(1) << 18;
__global__ void __launch_bounds__(kSqerrThreads) k_sqerr_single(const float* __restrict__ p,
                                                                const float* __restrict__ t, uint64_t n,
                                                                float* __restrict__ loss) {
    __shared__ float s[kSqerrThreads / 64];
    float acc = 0;
    uint64_t i0 = 0;
    if ((((uintptr_t)p | (uintptr_t)t) & 15) == 0) {
        // 128-bit loads over the first n - n % 4 elements (more loads in
        // flight per thread: the single block is latency-bound)
        const uint64_t n4 = n / 4;
        const float4* p4 = reinterpret_cast<const float4*>(p);
        const float4* t4 = reinterpret_cast<const float4*>(t);
#pragma unroll 4
        for (uint64_t i = threadIdx.x; i < n4; i += kSqerrThreads) {
            const float4 a = p4[i], b = t4[i];
            const float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
            acc += d0 * d0;
            acc += d1 * d1;
            acc += d2 * d2;
            acc += d3 * d3;
        }
        i0 = 4 * n4;
    }
    for (uint64_t i = i0 + threadIdx.x; i < n; i += kSqerrThreads) {
        const float d = p[i] - t[i];
        acc += d * d;
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (threadIdx.x % 64 == 0) s[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float tot = 0;
        for (int w = 0; w < kSqerrThreads / 64; w++) tot += s[w];
        loss[0] = tot / (float)n;  // rpl_core.c:457
    }
}

// rpl_core.c:441-444.  The update contracts to fma(g0 * factor, p - t, dp);
// overwrite uses +0.0 for dp, as a zeroed gradient would hold.
// g0p NULL: the root gradient's value is g0v (a gradient marked, not
// written, by tensor_backward).
__global__ void __launch_bounds__(kThreads) k_mse_backward(const float* __restrict__ p,
                                                           const float* __restrict__ t, uint64_t n,
                                                           const float* __restrict__ g0p, float g0v,
                                                           float* __restrict__ dp, int overwrite) {
    const float factor = 2.0f / (float)n;
    const float g0f = (g0p ? *g0p : g0v) * factor;
    GRID_STRIDE(i, n) { dp[i] = mse_grad_acc(overwrite ? 0.0f : dp[i], g0f, p[i], t[i]); }
}

// Activations of the device seam (tensor_sigmoid_gpu / tensor_tanh_gpu /
// tensor_gelu_gpu, src/rpl_gpu.c:437-522) with the reference's CPU formulas
// (tensor_sigmoid src/rpl_core.c:302-304, tensor_tanh_inplace :490-491,
// tensor_gelu_inplace :493-497) on the device's expf / tanhf / powf.  GCC
// contracts the GELU inner sum to fma(0.044715f, x^3, x); gelu_c is
// sqrtf(2/pi) as the reference computes it (passed in from the host).
enum Act { kSigmoid = 0, kTanh = 1, kGelu = 2 };
template <int ACT>
__global__ void __launch_bounds__(kThreads) k_act(const float* __restrict__ x, float* __restrict__ y, uint64_t n,
                                                  float gelu_c) {
#pragma clang fp contract(off)
    GRID_STRIDE(i, n) {
        const float v = x[i];
        float r;
        if constexpr (ACT == kSigmoid) {
            r = 1.0f / (1.0f + expf(-v));
        } else if constexpr (ACT == kTanh) {
            r = tanhf(v);
        } else {
            r = 0.5f * v * (1.0f + tanhf(gelu_c * __fmaf_rn(0.044715f, powf(v, 3.0f), v)));
        }
        y[i] = r;
    }
}

// optimizer_sgd_step (src/rpl_training.c:70-114), one element per thread.
// The reference's loops compile (GCC -O3, FMA) to these fused forms, which
// the oracle's golden vectors pin bit for bit:
//   g = fma(wd, p, g)                   weight decay (grad updated in place)
//   v = fma(mom, v, (1 - damp) * g)     momentum buffer
//   g = fma(mom, v, g)                  Nesterov (grad updated in place)
//   p = fma(-lr, d, p)                  d = g (Nesterov / no momentum) or v
// One element of optimizer_sgd_step (src/rpl_training.c:70-114).
__device__ __forceinline__ void sgd_one(float* __restrict__ p, float* __restrict__ g, float* __restrict__ v,
                                        uint64_t i, float lr, float mom, float keep, float wd, int nesterov) {
#pragma clang fp contract(off)
    const float pi = p[i];
    float gi = g[i];
    if (wd != 0.0f) gi = __fmaf_rn(wd, pi, gi);
    float d = gi;
    if (mom != 0.0f) {
        const float vi = __fmaf_rn(mom, v[i], keep * gi);
        v[i] = vi;
        if (nesterov) {
            gi = __fmaf_rn(mom, vi, gi);
            d = gi;
        } else {
            d = vi;
        }
    }
    g[i] = gi;
    p[i] = __fmaf_rn(-lr, d, pi);
}

// Several parameter tensors in one launch: tensor k gets the blocks
// [first[k], first[k+1]).
__global__ void __launch_bounds__(kThreads) k_sgd_multi(RplSgdTensors ts, float lr, float mom, float damp, float wd,
                                                        int nesterov) {
    int k = 0;
    while (k + 1 < ts.count && blockIdx.x >= ts.first[k + 1]) k++;
    const uint32_t b = blockIdx.x - ts.first[k], nb = ts.first[k + 1] - ts.first[k];
    const float keep = 1.0f - damp;
    for (uint64_t i = (uint64_t)b * kThreads + threadIdx.x; i < ts.n[k]; i += (uint64_t)nb * kThreads)
        sgd_one(ts.p[k], ts.g[k], ts.v[k], i, lr, mom, keep, wd, nesterov);
}

__global__ void __launch_bounds__(kThreads) k_sgd_step(float* __restrict__ p, float* __restrict__ g,
                                                       float* __restrict__ v, uint64_t n, float lr, float mom,
                                                       float damp, float wd, int nesterov) {
#pragma clang fp contract(off)
    const float keep = 1.0f - damp;
    GRID_STRIDE(i, n) {
        const float pi = p[i];
        float gi = g[i];
        if (wd != 0.0f) gi = __fmaf_rn(wd, pi, gi);
        float d = gi;
        if (mom != 0.0f) {
            const float vi = __fmaf_rn(mom, v[i], keep * gi);
            v[i] = vi;
            if (nesterov) {
                gi = __fmaf_rn(mom, vi, gi);
                d = gi;
            } else {
                d = vi;
            }
        }
        g[i] = gi;
        p[i] = __fmaf_rn(-lr, d, pi);
    }
}

}  // namespace

using namespace rplhip;

#define NEED(cond, name)                                                     \
    do {                                                                     \
        if (!(cond)) return fail(RPLHIP_ERR_INVALID, name ": NULL pointer"); \
    } while (0)

extern "C" {

int rplhip_add_broadcast(const float* a, const float* b, float* out, uint64_t n, uint64_t nb,
                         rplhip_stream_t stream) {
    return rplhip_bias_add_relu(a, b, out, nullptr, n, nb, stream);
}

int rplhip_bias_add_relu(const float* mm, const float* b, float* out, float* act, uint64_t n,
                         uint64_t nb, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(mm && b && out, "rplhip_bias_add_relu");
    if (nb == 0) return fail(RPLHIP_ERR_INVALID, "rplhip_bias_add_relu: broadcast size is 0");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_bias_add_relu, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), mm, b,
                       out, act, n, nb);
    return check_launch("bias_add_relu");
}

int rplhip_relu(const float* x, float* y, uint64_t n, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(x && y, "rplhip_relu");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_relu, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), x, y, n);
    return check_launch("relu");
}

int rplhip__relu_backward(const float* x, const float* dy, float* dx, uint64_t n, int overwrite,
                          rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(x && dy && dx, "rplhip_relu_backward");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_relu_backward, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), x, dy,
                       dx, n, overwrite);
    return check_launch("relu_backward");
}

int rplhip_relu_backward(const float* x, const float* dy, float* dx, uint64_t n,
                         rplhip_stream_t stream) {
    return rplhip__relu_backward(x, dy, dx, n, 0, stream);
}

int rplhip__accumulate(const float* dy, float* dx, uint64_t n, int overwrite, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(dy && dx, "rplhip_accumulate");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_accumulate, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), dy, dx, n,
                       overwrite);
    return check_launch("accumulate");
}

int rplhip_accumulate(const float* dy, float* dx, uint64_t n, rplhip_stream_t stream) {
    return rplhip__accumulate(dy, dx, n, 0, stream);
}

int rplhip_fill(float* x, uint64_t n, float value, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(x, "rplhip_fill");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_fill, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), x, n, value);
    return check_launch("fill");
}

int rplhip_bias_grad(const float* dy, uint64_t n, float* db, uint64_t nb, rplhip_stream_t stream) {
    return rplhip__bias_grad(dy, n, db, nb, 0, stream);
}

}  // extern "C"

namespace {
// Row splits of the bias-gradient reduction of dy [n / nb rows, nb].
struct ColsumPlan {
    uint64_t full_rows, cx, splits, rps;
};
ColsumPlan colsum_plan(uint64_t n, uint64_t nb) {
    ColsumPlan c;
    // backward_add's j-loop visits i, i+nb, ... < n: ceil(n/nb) rows.
    c.full_rows = (n + nb - 1) / nb;
    c.cx = (nb + kColTile - 1) / kColTile;
    // Enough row splits to put ~4 blocks on every CU, each split >= 16 rows
    // (4 rows per thread: one batch of loads).
    uint64_t want = (4ull * cu_count() + c.cx - 1) / c.cx;
    uint64_t splits = c.full_rows / 16;
    if (splits > want) splits = want;
    if (splits < 1) splits = 1;
    if (splits > 65535) splits = 65535;
    c.rps = (c.full_rows + splits - 1) / splits;
    splits = (c.full_rows + c.rps - 1) / c.rps;
    c.splits = splits < 1 ? 1 : splits;
    return c;
}
}  // namespace

extern "C" {

int rplhip__bias_grad(const float* dy, uint64_t n, float* db, uint64_t nb, int overwrite, rplhip_stream_t stream) {
    if (nb == 0) return RPLHIP_OK;
    NEED(dy && db, "rplhip_bias_grad");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    const ColsumPlan c = colsum_plan(n, nb);
    void* ws = nullptr;
    int st = ws_alloc(&ws, sizeof(float) * c.splits * nb, s);
    if (st) return st;
    // A ragged last row (n % nb != 0, columns < n % nb get one more term) is
    // handled by the r*nb + c < n bound in the partial kernel.
    hipLaunchKernelGGL((k_colsum_partial<false, kSrcGrad>), dim3((unsigned)c.cx, (unsigned)c.splits), dim3(kThreads),
                       0, s, dy, n, c.full_rows, nb, c.rps, (float*)ws, (float*)nullptr, 0, RplGradSrc{});
    hipLaunchKernelGGL(k_colsum_finish, dim3((unsigned)((nb + kFinCols - 1) / kFinCols)), dim3(kThreads), 0, s,
                       (const float*)ws, (int)c.splits,
                       nb, db, overwrite);
    st = check_launch("bias_grad");
    ws_free(ws, s);
    return st;
}

int rplhip__add_backward_begin(const float* dy, uint64_t n, float* dx, int dx_overwrite, uint64_t nb,
                               const RplGradSrc* src, RplColsum* cs, rplhip_stream_t stream) {
    cs->ws = nullptr;
    cs->splits = 0;
    cs->nb = nb;
    if (n == 0) return RPLHIP_OK;
    const int kind = src ? src->kind : kSrcGrad;
    NEED(dx && (kind == kSrcGrad ? dy != nullptr : src->x && src->y && src->g), "rplhip_add_backward");
    NEED(kind == kSrcGrad || kind == kSrcRelu || kind == kSrcMse, "rplhip_add_backward (source)");
    if (nb == 0) {
        NEED(kind == kSrcGrad, "rplhip_add_backward (fused source without a bias)");
        return rplhip__accumulate(dy, dx, n, dx_overwrite, stream);
    }
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    const ColsumPlan c = colsum_plan(n, nb);
    int st = ws_alloc(&cs->ws, sizeof(float) * c.splits * nb, s);
    if (st) return st;
    cs->splits = c.splits;
    const dim3 grid((unsigned)c.cx, (unsigned)c.splits);
    const RplGradSrc sv = src ? *src : RplGradSrc{};
    if (kind == kSrcRelu)
        hipLaunchKernelGGL((k_colsum_partial<true, kSrcRelu>), grid, dim3(kThreads), 0, s, dy, n, c.full_rows, nb,
                           c.rps, (float*)cs->ws, dx, dx_overwrite, sv);
    else if (kind == kSrcMse)
        hipLaunchKernelGGL((k_colsum_partial<true, kSrcMse>), grid, dim3(kThreads), 0, s, dy, n, c.full_rows, nb,
                           c.rps, (float*)cs->ws, dx, dx_overwrite, sv);
    else
        hipLaunchKernelGGL((k_colsum_partial<true, kSrcGrad>), grid, dim3(kThreads), 0, s, dy, n, c.full_rows, nb,
                           c.rps, (float*)cs->ws, dx, dx_overwrite, sv);
    st = check_launch("add_backward");
    if (st) {
        ws_free(cs->ws, s);
        cs->ws = nullptr;
    }
    return st;
}

int rplhip__add_backward_finish(RplColsum* cs, float* db, int db_overwrite, rplhip_stream_t stream) {
    if (!cs->ws) return RPLHIP_OK;
    hipStream_t s = as_stream(stream);
    int st = RPLHIP_OK;
    if (db) {
        hipLaunchKernelGGL(k_colsum_finish, dim3((unsigned)((cs->nb + kFinCols - 1) / kFinCols)), dim3(kThreads), 0,
                           s, (const float*)cs->ws, (int)cs->splits, cs->nb, db, db_overwrite);
        st = check_launch("add_backward (bias)");
    }
    ws_free(cs->ws, s);
    cs->ws = nullptr;
    return st;
}

int rplhip_mse_loss(const float* pred, const float* target, uint64_t n, float* loss,
                    rplhip_stream_t stream) {
    NEED(pred && target && loss, "rplhip_mse_loss");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (n <= kSqerrSingleMax) {
        hipLaunchKernelGGL(k_sqerr_single, dim3(1), dim3(kSqerrThreads), 0, s, pred, target, n, loss);
        return check_launch("mse_loss");
    }
    int g = grid_for(n);
    if (g > 1024) g = 1024;
    void* ws = nullptr;
    int st = ws_alloc(&ws, sizeof(float) * g, s);
    if (st) return st;
    hipLaunchKernelGGL(k_sqerr_partial, dim3(g), dim3(kThreads), 0, s, pred, target, n, (float*)ws);
    hipLaunchKernelGGL(k_sqerr_finish, dim3(1), dim3(kThreads), 0, s, (const float*)ws, g, n, loss);
    st = check_launch("mse_loss");
    ws_free(ws, s);
    return st;
}

int rplhip__mse_backward(const float* pred, const float* target, uint64_t n, const float* g0, float g0_value,
                         float* dpred, int overwrite, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(pred && target && dpred, "rplhip_mse_backward");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_mse_backward, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), pred,
                       target, n, g0, g0_value, dpred, overwrite);
    return check_launch("mse_backward");
}

int rplhip_mse_backward(const float* pred, const float* target, uint64_t n, const float* g0,
                        float* dpred, rplhip_stream_t stream) {
    if (!g0) return fail(RPLHIP_ERR_INVALID, "rplhip_mse_backward: NULL pointer");
    return rplhip__mse_backward(pred, target, n, g0, 0.0f, dpred, 0, stream);
}

static int launch_act(int act, const float* x, float* y, uint64_t n, rplhip_stream_t stream, const char* what) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !y) return fail(RPLHIP_ERR_INVALID, "%s: NULL pointer", what);
    RPLHIP_REQUIRE_DEVICE();
    const float gelu_c = sqrtf((float)(2.0 / M_PI));  // host libm: correctly rounded, as the reference's
    const dim3 g(grid_for(n)), b(kThreads);
    if (act == kSigmoid)
        hipLaunchKernelGGL(k_act<kSigmoid>, g, b, 0, as_stream(stream), x, y, n, gelu_c);
    else if (act == kTanh)
        hipLaunchKernelGGL(k_act<kTanh>, g, b, 0, as_stream(stream), x, y, n, gelu_c);
    else
        hipLaunchKernelGGL(k_act<kGelu>, g, b, 0, as_stream(stream), x, y, n, gelu_c);
    return check_launch(what);
}

int rplhip_sigmoid(const float* x, float* y, uint64_t n, rplhip_stream_t stream) {
    return launch_act(kSigmoid, x, y, n, stream, "rplhip_sigmoid");
}

int rplhip_tanh(const float* x, float* y, uint64_t n, rplhip_stream_t stream) {
    return launch_act(kTanh, x, y, n, stream, "rplhip_tanh");
}

int rplhip_gelu(const float* x, float* y, uint64_t n, rplhip_stream_t stream) {
    return launch_act(kGelu, x, y, n, stream, "rplhip_gelu");
}

int rplhip_sgd_step(float* param, float* grad, float* velocity, uint64_t n, float lr, float momentum,
                    float dampening, float weight_decay, int nesterov, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    NEED(param && grad && (momentum == 0.0f || velocity), "rplhip_sgd_step");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_sgd_step, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), param, grad, velocity, n,
                       lr, momentum, dampening, weight_decay, nesterov);
    return check_launch("sgd_step");
}

int rplhip__sgd_step_multi(RplSgdTensors* ts, float lr, float momentum, float dampening, float weight_decay,
                           int nesterov, rplhip_stream_t stream) {
    if (ts->count <= 0) return RPLHIP_OK;
    if (ts->count > RPL_SGD_MULTI) return fail(RPLHIP_ERR_INVALID, "rplhip_sgd_step_multi: %d tensors", ts->count);
    RPLHIP_REQUIRE_DEVICE();
    uint32_t blocks = 0;
    for (int k = 0; k < ts->count; k++) {
        NEED(ts->p[k] && ts->g[k] && (momentum == 0.0f || ts->v[k]), "rplhip_sgd_step_multi");
        ts->first[k] = blocks;
        blocks += (uint32_t)grid_for(ts->n[k] ? ts->n[k] : 1);
    }
    ts->first[ts->count] = blocks;
    hipLaunchKernelGGL(k_sgd_multi, dim3(blocks), dim3(kThreads), 0, as_stream(stream), *ts, lr, momentum, dampening,
                       weight_decay, nesterov);
    return check_launch("sgd_step_multi");
}

}  // extern "C"
