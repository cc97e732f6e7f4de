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

// Descending bitonic network over n 64-bit composites (unique keys give a
// strict order) held in registers: thread t holds
// elements t*E .. t*E+E-1 (threads at or past n / E hold none and only join
// the barriers).  Pairs (e, e ^ j) inside a thread swap registers, pairs
// inside a wave meet through lane permutes, and pairs across waves through
// LDS, two buffers used in turn with one barrier per such step: of the 66
// steps of a 2048-key network, 6 cross waves.  Every pair costs one 64-bit
// compare; which of the two an element keeps (the larger where its half of
// the run sorts descending) is fixed per thread for the steps with j >= E,
// since e & j and e & k then do not depend on the element's index within the
// thread.
// (the larger of a, b where keep_max, else the smaller; a == b keeps a)
__device__ __forceinline__ uint64_t bitonic_keep(uint64_t a, uint64_t b, bool keep_max) {
    return ((a < b) == keep_max) ? b : a;
}

template <int E, int J>
__device__ __forceinline__ void step_in_thread(uint64_t (&v)[E], int e0, int k, bool last) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
        if ((i & J) == 0) {
            const bool desc = last || (((e0 + i) & k) == 0);
            const uint64_t a = v[i], b = v[i + J];
            const bool swap = (a < b) == desc;
            v[i] = swap ? b : a;
            v[i + J] = swap ? a : b;
        }
    }
}

// Every aligned run of `group` (a power of two dividing n) is sorted on its
// own; group = n sorts the whole set.
template <int E>
__device__ __forceinline__ void bitonic_desc_regs(uint64_t (&v)[E], int n, uint64_t* buf0, uint64_t* buf1, int group) {
    const int e0 = (int)threadIdx.x * E;
    const int lane = (int)(threadIdx.x & (kWave - 1));
    const bool live = e0 < n;
    int flip = 0;
    for (int k = 2; k <= group; k <<= 1) {
        const bool last = k == group;
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j < E) {
                if (j == 1) step_in_thread<E, 1>(v, e0, k, last);
                if (E > 2 && j == 2) step_in_thread<E, (E > 2 ? 2 : 1)>(v, e0, k, last);
                if (E > 4 && j == 4) step_in_thread<E, (E > 4 ? 4 : 1)>(v, e0, k, last);
                if (E > 8 && j == 8) step_in_thread<E, (E > 8 ? 8 : 1)>(v, e0, k, last);
                continue;
            }
            // (j >= E: the same for every element of the thread)
            const bool keep_max = ((e0 & j) == 0) == (last || (e0 & k) == 0);
            if (j / E < kWave) {
                const int addr = (lane ^ (j / E)) << 2;  // partner lane, as ds_bpermute's byte address
#pragma unroll
                for (int i = 0; i < E; ++i) {
                    const uint64_t a = v[i];
                    const uint32_t blo = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)(uint32_t)a);
                    const uint32_t bhi = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)(uint32_t)(a >> 32));
                    v[i] = bitonic_keep(a, ((uint64_t)bhi << 32) | blo, keep_max);
                }
            } else {
                uint64_t* w = flip ? buf1 : buf0;
                flip ^= 1;
                if (live)
#pragma unroll
                    for (int i = 0; i < E; ++i) w[e0 + i] = v[i];
                __syncthreads();
                if (live)
#pragma unroll
                    for (int i = 0; i < E; ++i) v[i] = bitonic_keep(v[i], w[(e0 + i) ^ j], keep_max);
            }
        }
    }
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
