// Shared helpers for the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rplhip.h"

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

namespace rplhip {

// Set the thread-local error string and return `code`.
int fail(int code, const char* fmt, ...);
// Lazily initialise the device; returns RPLHIP_OK or an error status.
int ensure_device();
// Check the last launch; returns RPLHIP_OK or RPLHIP_ERR_HIP.
int check_launch(const char* what);
// Stream-ordered temporary device memory (hipMallocAsync on `stream`).
int ws_alloc(void** p, size_t bytes, hipStream_t stream);
void ws_free(void* p, hipStream_t stream);
// Number of compute units of the current device.
int cu_count();

inline hipStream_t as_stream(rplhip_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace rplhip

#define RPLHIP_REQUIRE_DEVICE()                          \
    do {                                                 \
        int _st = rplhip::ensure_device();               \
        if (_st != RPLHIP_OK) return _st;                \
    } while (0)

#define RPLHIP_CHECK(call)                                                              \
    do {                                                                                \
        hipError_t _e = (call);                                                         \
        if (_e != hipSuccess)                                                           \
            return rplhip::fail(RPLHIP_ERR_HIP, "%s failed: %s", #call,                 \
                                hipGetErrorString(_e));                                 \
    } while (0)

namespace rplhip {
// Tile index -> (tile_m, tile_n) for a 1-D grid of tm x tn tiles:
// 1. undo the round-robin XCD dispatch (block b runs on XCD b % 8) so that
//    each XCD owns a contiguous range of virtual tile indices;
// 2. walk that range in groups of kGroupM tile-rows, column by column.
constexpr uint32_t kXcds = 8, kGroupM = 8;  // MI355X: 8 XCDs of 32 CUs

__device__ __forceinline__ void tile_of(uint32_t b, uint32_t tm, uint32_t tn, uint32_t& im, uint32_t& in) {
    const uint32_t T = tm * tn;
    const uint32_t q = T / kXcds, r = T % kXcds;
    const uint32_t x = b % kXcds, idx = b / kXcds;
    const uint32_t t = x * q + (x < r ? x : r) + idx;
    const uint32_t group = kGroupM * tn;
    const uint32_t g = t / group, first = g * kGroupM;
    const uint32_t gm = tm - first < kGroupM ? tm - first : kGroupM;
    const uint32_t w = t - g * group;
    im = first + w % gm;
    in = w / gm;
}

}  // namespace rplhip

// x86-64 cvttss2si: truncation toward zero; NaN and values outside
// [-2^31, 2^31) give INT32_MIN.  The reference's (int32_t) casts of roundf
// results compile to it, and its outcome is part of the observable contract
// (e.g. an all-zero tensor has scale 0, 0/0 = NaN, and quantizes to -128).
__device__ __forceinline__ int32_t x86_cvt_i32(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}

// x86_cvt_i32(roundf(y)) for every float y, in four VALU operations:
// roundf(y) == trunc(y + copysign(0.49999997f, y)) when the sum is rounded
// to nearest-even (0.49999997f is the float just below 0.5), and the range
// test on the sum is the range test on the rounded value.  Checked against
// glibc roundf + cvttss2si for all 2^32 floats (tests/test_round_identity.py).
// The add must stay a separately rounded operation, never an FMA with the
// product that feeds it, hence contract(off) here and in its callers.
__device__ __forceinline__ int32_t x86_round_cvt(float y) {
#pragma clang fp contract(off)
    const float t = y + __builtin_copysignf(0.49999997f, y);
    return (t >= -2147483648.0f && t < 2147483648.0f) ? (int32_t)t : INT32_MIN;
}

// Wrapping int32 add (the reference's signed adds wrap on x86).
__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}
__device__ __forceinline__ int32_t wrap_mul(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a * (uint32_t)b);
}

// q = clamp(x86((int32)roundf(x / scale)) + zp, -128, 127)
// (src/rpl_core.c:523-526; IEEE division: hipcc keeps fp32 division
// correctly rounded unless told otherwise, and roundf rounds ties away
// from zero).
__device__ __forceinline__ int8_t quantize_one(float x, float scale, int32_t zp) {
    int32_t v = wrap_add(x86_cvt_i32(roundf(x / scale)), zp);
    v = v < -128 ? -128 : (v > 127 ? 127 : v);
    return (int8_t)v;
}
