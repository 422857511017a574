// Elementwise codecs next to quantization: the QAT fake-quant step
// (src/rpl_quantization.c:195-237) and the FP16 codec (src/rpl_half.c:10-75),
// bit-exact with the reference.
#include "common.h"

namespace {

constexpr int kThreads = 256;

inline uint32_t grid_for(uint64_t n) {
    const uint64_t g = (n + kThreads - 1) / kThreads;
    return (uint32_t)(g < 65536 ? g : 65536);  // grid-stride loops cover the rest
}

// q = clamp((int32)roundf(x * inv_scale + zp), -128, 127); y = (q - zp) *
// scale.  GCC contracts x * inv_scale + zp to fma(x, inv_scale, zp).
__global__ void __launch_bounds__(kThreads) k_fake_quant(const float* __restrict__ x, float* __restrict__ y,
                                                         uint64_t n, float inv_scale, float zp, float scale) {
#pragma clang fp contract(off)
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kThreads) {
        int32_t q = x86_round_cvt(__fmaf_rn(x[i], inv_scale, zp));
        q = q < -128 ? -128 : (q > 127 ? 127 : q);
        y[i] = ((float)q - zp) * scale;
    }
}

// float_to_half_impl: truncates the mantissa; zero / subnormal inputs and
// results below the half range give +-0; overflow gives +-inf; NaN gives a
// quiet NaN with mantissa 0x200.
__global__ void __launch_bounds__(kThreads) k_f32_to_half(const float* __restrict__ x, uint16_t* __restrict__ h,
                                                          uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kThreads) {
        const uint32_t f = __float_as_uint(x[i]);
        const uint32_t exp = (f >> 23) & 0xFF, mant = f & 0x7FFFFF;
        uint32_t he = 0, hm = 0;
        if (exp == 255) {
            he = 31;
            hm = mant ? 0x200 : 0;
        } else if (exp != 0) {
            const int e = (int)exp - 127 + 15;
            if (e >= 31) {
                he = 31;
            } else if (e > 0) {
                he = (uint32_t)e;
                hm = mant >> 13;
            }
        }
        h[i] = (uint16_t)(((f >> 31) << 15) | (he << 10) | hm);
    }
}

// half_to_float_impl: subnormal halves give +-0; inf / NaN keep their class
// (NaN mantissa 0x7FFFFF).
__global__ void __launch_bounds__(kThreads) k_half_to_f32(const uint16_t* __restrict__ h, float* __restrict__ x,
                                                          uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kThreads) {
        const uint32_t v = h[i];
        const uint32_t exp = (v >> 10) & 0x1F, mant = v & 0x3FF;
        uint32_t fe, fm;
        if (exp == 31) {
            fe = 255;
            fm = mant ? 0x7FFFFF : 0;
        } else if (exp == 0) {
            fe = 0;
            fm = 0;
        } else {
            fe = exp + 127 - 15;
            fm = mant << 13;
        }
        x[i] = __uint_as_float(((v >> 15) << 31) | (fe << 23) | fm);
    }
}

}  // namespace

using namespace rplhip;

extern "C" {

int rplhip_fake_quant(const float* x, float* y, uint64_t n, float scale, float zero_point, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !y) return fail(RPLHIP_ERR_INVALID, "rplhip_fake_quant: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    const float inv_scale = 1.0f / scale;  // IEEE division, as the reference
    hipLaunchKernelGGL(k_fake_quant, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), x, y, n, inv_scale,
                       zero_point, scale);
    return check_launch("fake_quant");
}

int rplhip_float_to_half(const float* x, uint16_t* h, uint64_t n, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !h) return fail(RPLHIP_ERR_INVALID, "rplhip_float_to_half: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_f32_to_half, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), x, h, n);
    return check_launch("float_to_half");
}

int rplhip_half_to_float(const uint16_t* h, float* x, uint64_t n, rplhip_stream_t stream) {
    if (n == 0) return RPLHIP_OK;
    if (!x || !h) return fail(RPLHIP_ERR_INVALID, "rplhip_half_to_float: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    hipLaunchKernelGGL(k_half_to_f32, dim3(grid_for(n)), dim3(kThreads), 0, as_stream(stream), h, x, n);
    return check_launch("half_to_float");
}

}  // extern "C"
