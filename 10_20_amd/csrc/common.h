// Shared helpers for the gfx950 kernels of libv1idx: status/error plumbing,
// launch checks, order-preserving float keys and wave64 primitives.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <stdarg.h>
#include <stdio.h>
#include "../../include/v1idx.h"

namespace v1 {

// ---------------------------------------------------------------- host side
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);

#define V1_REQUIRE(cond, ...)                  \
    do {                                       \
        if (!(cond)) {                         \
            ::v1::set_error(__VA_ARGS__);      \
            return V1_ERR_INVALID;             \
        }                                      \
    } while (0)

// Checks the launch that was just issued (configuration errors surface here).
#define V1_LAUNCHED(what) ::v1::hip_status(hipGetLastError(), what)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Device-wide primitives (sort64.hip) shared by the batched page manager.
// sort_pairs: stable ascending sort of (uint64 key, uint32 value) pairs.
int64_t sort_pairs_workspace(int64_t n);
int sort_pairs(const uint64_t* keys, const uint32_t* vals, uint64_t* keys_out, uint32_t* vals_out, int64_t n,
               int key_bits, void* ws, int64_t ws_bytes, hipStream_t st, const char* name);
// scan_exclusive: out[i] = sum of in[0..i), *total = sum of all (device pointers).
int64_t scan_workspace(int64_t n);
int scan_exclusive(const uint32_t* in, uint32_t* out, uint32_t* total, int64_t n, void* ws, int64_t ws_bytes,
                   hipStream_t st, const char* name);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device; 256 if unknown).
inline int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        cus[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : 256;
    }
    return cus[dev];
}

// ---------------------------------------------------------------- device side
constexpr int kWave = 64;

// Order-preserving map of an fp32 score onto uint32: a > b  <=>  key(a) > key(b).
// -0.0 is folded onto +0.0 so that the two compare equal (IEEE semantics).
__device__ __forceinline__ uint32_t score_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_score(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Inclusive prefix sum over the 64 lanes of a wave, on DPP lane moves:
// row_shr 1/2/4/8 scans each 16-lane row, then row_bcast15 / row_bcast31 carry
// the row totals into rows 1,3 and 2,3.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ uint32_t popc64(uint64_t m) { return (uint32_t)__popcll(m); }

// Number of set bits of `m` strictly below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    const uint32_t lane = __lane_id();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    return popc64(m & below);
}

// Exact n / d whenever n * d < 2^32, with m = ceil(2^32 / d) and d >= 2
// (d = 1 would need m = 2^32).
__device__ __forceinline__ uint32_t small_div(uint32_t n, uint32_t m) { return __umulhi(n, m); }

inline uint32_t small_div_magic(uint32_t d) {
    return (uint32_t)((((uint64_t)1 << 32) + d - 1) / d);
}

// OCP e4m3fn byte -> float (exact; codes 0x7f / 0xff, NaN in the format, read
// as +-480, which no encoder here produces).
__device__ __forceinline__ float e4m3_value(uint32_t c) {
    const uint32_t e = (c >> 3) & 15, m = c & 7;
    const float v = e == 0 ? (float)m * 0.001953125f : __builtin_ldexpf((float)(8 + m), (int)e - 10);
    return (c & 0x80) ? -v : v;
}

// Round-to-nearest-even encoding of |x| <= 448 as OCP e4m3fn.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
    const float a = fabsf(x);
    uint32_t code;
    if (a < 0.015625f) {  // below 2^-6: subnormal quanta of 2^-9 (8 quanta = the first normal)
        code = (uint32_t)rintf(a * 512.0f);
    } else {
        int e;
        frexpf(a, &e);  // a = f * 2^e, f in [0.5, 1)
        e -= 1;         // a in [2^e, 2^(e+1))
        const uint32_t m = (uint32_t)rintf(__builtin_ldexpf(a, -e) * 8.0f - 8.0f);  // 0..8
        code = (uint32_t)((e + 7) << 3) + m;  // m == 8 carries into the exponent
    }
    return code | (x < 0.f ? 0x80u : 0u);
}

}  // namespace v1
