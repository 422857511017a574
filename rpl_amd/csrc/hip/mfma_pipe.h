// Building blocks of the direct-to-LDS MFMA pipelines (gemm_i8.hip,
// gemm_f32.hip): compile-time loops, the LDS row swizzle, wave-uniform
// buffer resources and s_waitcnt immediates.
#pragma once

#include <type_traits>

#include "common.h"

namespace rplhip {

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 at compile time.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// LDS tiles of 64-byte rows store the four 16-byte chunks of row r
// XOR-swizzled (chunk c at slot c ^ swz(r)).  The fragment reads have lane l
// read row l%32 (plus a multiple of 32) at one chunk per half-wave; measured
// on gfx950 (SQ_LDS_BANK_CONFLICT per ds_read_b128), this swizzle reads them
// without bank conflicts, as do (r>>2)&3, (r>>3)&3 and (r^(r>>2))&3, while
// ((r>>1)^(r>>3))&3 and (r>>1)&3 cost 4 extra cycles per read and no
// swizzle 12.  The function must depend on r % 32 only (rows 32 apart share
// lanes).  Tile writes fill whole 64-byte rows, which any row-local
// permutation leaves conflict-free.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// Word 3 of a raw buffer resource on gfx950 (32-bit data format, no
// swizzle, range-checked against num_records).
constexpr int kBufferFlags = 0x00020000;

// Raw buffer resource for `bytes` bytes at `base`.  The fields go through
// readfirstlane so the resource is provably wave-uniform and lives in SGPRs:
// a resource the compiler cannot prove uniform makes it wrap every buffer
// access in a readfirstlane/compare/exec loop.  Callers pass values that are
// uniform already (derived from blockIdx and kernel arguments).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, (int)n, kBufferFlags);
}

// gfx9 s_waitcnt immediate: vmcnt in bits [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8]; a field at its maximum does not wait.
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8); }

typedef __attribute__((address_space(3))) void* lds_ptr;

}  // namespace rplhip
