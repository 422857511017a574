// Scaled dot-product attention (src/rpl_attention.c:16-111) on the device:
// QK^T and PV on the FP32 GEMMs of gemm_f32.hip (one launch per batch
// entry, operands addressed in place), and between them a masked softmax
// with one wave per row of scores.
#include <float.h>
#include <math.h>

#include "common.h"

namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row

// Row r of S [rows, n]: s = mask[r*n+j] == 0 ? -1e9 : s, then
// s = exp(s - max) / sum (the reference's order: max, exp and sum, divide).
__global__ void __launch_bounds__(64 * kRowsPerBlock) k_masked_softmax(float* __restrict__ S,
                                                                       const float* __restrict__ mask,
                                                                       uint64_t rows, uint32_t n) {
    const uint64_t r = (uint64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / 64;
    const uint32_t lane = threadIdx.x % 64;
    if (r >= rows) return;
    float* row = S + r * n;
    const float* mrow = mask ? mask + r * n : nullptr;
    float mx = -FLT_MAX;
    for (uint32_t j = lane; j < n; j += 64) {
        float v = row[j];
        if (mrow && mrow[j] == 0.0f) {
            v = -1e9f;
            row[j] = v;
        }
        mx = fmaxf(mx, v);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.0f;
    for (uint32_t j = lane; j < n; j += 64) {
        const float e = expf(row[j] - mx);
        row[j] = e;
        sum += e;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    for (uint32_t j = lane; j < n; j += 64) row[j] = row[j] / sum;
}

}  // namespace

using namespace rplhip;

extern "C" int rplhip_attention(const float* Q, const float* K, const float* V, const float* mask, float* out,
                                uint32_t B, uint32_t Sq, uint32_t Sk, uint32_t dk, uint32_t dv,
                                rplhip_stream_t stream) {
    if (B == 0 || Sq == 0 || dv == 0) return RPLHIP_OK;
    if (!out || (Sk && (!Q || !K || !V)) || (Sk && dk == 0))
        return fail(RPLHIP_ERR_INVALID, "rplhip_attention: NULL pointer or dk == 0");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t s = as_stream(stream);
    if (Sk == 0) return rplhip_fill(out, (uint64_t)B * Sq * dv, 0.0f, stream);
    const uint64_t n_scores = (uint64_t)B * Sq * Sk;
    void* ws = nullptr;
    int st = ws_alloc(&ws, n_scores * sizeof(float), s);
    if (st) return st;
    float* S = static_cast<float*>(ws);
    const float scale = 1.0f / sqrtf((float)dk);  // as the reference computes it
    // Per-batch score matrices big enough for the large-tile GEMM go one by
    // one through rplhip_sgemm (which reads C: start from zeros); the rest
    // take one batched launch per product that writes C without reading it.
    const bool big = (uint64_t)((Sq + 255) / 256) * ((Sk + 255) / 256) >= 2ull * cu_count() && dk % 16 == 0;
    if (big) {
        st = rplhip_fill(S, n_scores, 0.0f, stream);
        for (uint32_t b = 0; b < B && !st; b++)
            st = rplhip_sgemm(0, 1, Sq, Sk, dk, scale, Q + (uint64_t)b * Sq * dk, dk, K + (uint64_t)b * Sk * dk, dk,
                              0.0f, S + (uint64_t)b * Sq * Sk, Sk, stream);
    } else {
        st = rplhip_sgemm_batched(0, 1, Sq, Sk, dk, scale, Q, dk, (uint64_t)Sq * dk, K, dk, (uint64_t)Sk * dk, 0.0f,
                                  S, Sk, (uint64_t)Sq * Sk, B, 0, stream);
    }
    if (!st) {
        const uint64_t rows = (uint64_t)B * Sq;
        hipLaunchKernelGGL(k_masked_softmax, dim3((uint32_t)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                           dim3(64 * kRowsPerBlock), 0, s, S, mask, rows, Sk);
        st = check_launch("attention softmax");
    }
    const bool big_pv = (uint64_t)((Sq + 255) / 256) * ((dv + 255) / 256) >= 2ull * cu_count() && Sk % 16 == 0;
    if (big_pv) {
        if (!st) st = rplhip_fill(out, (uint64_t)B * Sq * dv, 0.0f, stream);
        for (uint32_t b = 0; b < B && !st; b++)
            st = rplhip_sgemm(0, 0, Sq, dv, Sk, 1.0f, S + (uint64_t)b * Sq * Sk, Sk, V + (uint64_t)b * Sk * dv, dv,
                              0.0f, out + (uint64_t)b * Sq * dv, dv, stream);
    } else if (!st) {
        st = rplhip_sgemm_batched(0, 0, Sq, dv, Sk, 1.0f, S, Sk, (uint64_t)Sq * Sk, V, dv, (uint64_t)Sk * dv, 0.0f,
                                  out, dv, (uint64_t)Sq * dv, B, 0, stream);
    }
    ws_free(ws, s);
    return st;
}
