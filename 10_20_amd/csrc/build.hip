// Index-build producer: the unit vectors, balanced cosine bisection and page
// assembly that turn a 1024-token bucket (16 native pages) into the permuted
// pages, member map and FP8 centers the query path reads.
//
// Semantics: sglang/srt/layers/attention/v1_deepseek/kernels.py:9-54
// (initialize, assemble), sglang/srt/layers/attention/v1_native/
// fused_grouping.py:38-61 (_dots, _anchor; _sort lives in sort64.hip / the
// group sort), chain order runtime.py:171-216.
//
// Arithmetic (this build's contract; the reference's Triton reductions have no
// specified order): every 128-wide fp32 sum keeps four partial sums over dims
// d = r (mod 4), each in ascending d with one rounding per product and per
// addition (no fused multiply-add), then (p0 + p1) + (p2 + p3).  Unit vectors
// are u_d = c_d * f with f = s / max(sqrt(sum (c_d s)^2), 1e-12), c_d the FP8
// key and s its scale.  Center means add the 8 members in order, times 1/8.
//
// Two forms: per-kernel drop-ins with the reference's launch shapes, and one
// fused kernel that builds a batch of buckets, one 1024-thread work-group per
// bucket (thread = position in the bucket's order): the token's FP8 key stays
// in registers, the group anchors go through LDS, each group's argmin is a
// wave reduction plus one LDS atomic per wave, and the stable sort of a group
// is a rank count over the group's (key, position) words.
#include "common.h"

// No contraction in this file: every product and every sum written here rounds
// on its own (plain operators: the header's __f*_rn helpers are compiled with
// contraction on and fuse once inlined), and sqrtf / division are correctly
// rounded with the HIP defaults.
#pragma clang fp contract(off)

namespace v1 {
namespace {

constexpr int kTokens = 1024;
constexpr int kWords = 32;                      // 128 FP8 bytes per token
constexpr int kPageWords = V1_PAGE_BYTES / 4;   // 2112
constexpr int kScaleWord = 2048;                // first scale word of a page

// FP8 byte r (0..3) of a packed word, as fp32 (exact).
template <int R>
__device__ __forceinline__ float fp8_at(uint32_t w) {
    return __builtin_amdgcn_cvt_f32_fp8((int)w, R);
}

// The four-partial 128-wide sum.
struct Acc4 {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    __device__ __forceinline__ void add(float p0, float p1, float p2, float p3) {
        a0 = (a0 + p0);
        a1 = (a1 + p1);
        a2 = (a2 + p2);
        a3 = (a3 + p3);
    }
    __device__ __forceinline__ float total() const { return ((a0 + a1) + (a2 + a3)); }
};

// Unit factor f of a token: s / max(||x||, 1e-12), x_d = c_d * s.
__device__ __forceinline__ float unit_factor(const uint32_t (&c)[kWords], float s) {
    Acc4 acc;
#pragma unroll
    for (int w = 0; w < kWords; ++w) {
        const float x0 = (fp8_at<0>(c[w]) * s), x1 = (fp8_at<1>(c[w]) * s);
        const float x2 = (fp8_at<2>(c[w]) * s), x3 = (fp8_at<3>(c[w]) * s);
        acc.add((x0 * x0), (x1 * x1), (x2 * x2), (x3 * x3));
    }
    return s / fmaxf(sqrtf(acc.total()), 1e-12f);
}

__device__ __forceinline__ void load_key(const uint8_t* row, uint32_t (&c)[kWords]) {
    const uint4* src = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) {
        const uint4 v = src[i];
        c[4 * i] = v.x;
        c[4 * i + 1] = v.y;
        c[4 * i + 2] = v.z;
        c[4 * i + 3] = v.w;
    }
}

// Power of two >= fl(max(amax, 1e-4) / 448): the smallest such.
__device__ __forceinline__ float center_scale(float amax) {
    const float v = fmaxf(amax, 1e-4f) / 448.0f;
    int e;
    const float m = frexpf(v, &e);
    return __builtin_ldexpf(1.0f, m == 0.5f ? e - 1 : e);
}

// ------------------------------------------------------------ drop-ins
// kernels.py:9-30: 16 tokens per program.
__global__ __launch_bounds__(64) void initialize_kernel(const uint8_t* __restrict__ K, const float* __restrict__ KS,
                                                        const int32_t* __restrict__ table, const int32_t* meta,
                                                        float* __restrict__ unit, int32_t* __restrict__ perm,
                                                        int32_t* flag) {
    const int32_t active = meta[2];
    if (blockIdx.x == 0 && threadIdx.x == 0) *flag = active != 0 ? -1 : 0;
    if (!active || threadIdx.x >= 16) return;
    const int32_t i = blockIdx.x * 16 + threadIdx.x;
    const int64_t page = table[i / 64];
    const int32_t slot = i % 64;
    uint32_t c[kWords];
    load_key(K + page * V1_PAGE_BYTES + slot * 128, c);
    const float s = KS[page * kPageWords + kScaleWord + slot];
    const float f = unit_factor(c, s);
    float4* dst = reinterpret_cast<float4*>(unit + (int64_t)i * 128);
#pragma unroll
    for (int w = 0; w < kWords; ++w)
        dst[w] = make_float4((fp8_at<0>(c[w]) * f), (fp8_at<1>(c[w]) * f),
                             (fp8_at<2>(c[w]) * f), (fp8_at<3>(c[w]) * f));
    perm[i] = i;
}

// fused_grouping.py:38-52: 16 positions per program, head = blockIdx.y.
__global__ __launch_bounds__(64) void dots_kernel(const float* __restrict__ U, const int32_t* __restrict__ P,
                                                  const int32_t* __restrict__ A, float* S, const int32_t* flag,
                                                  int32_t N, int32_t start, int32_t mode) {
    if (*flag >= 0 || threadIdx.x >= 16) return;
    const int32_t i = blockIdx.x * 16 + threadIdx.x, h = blockIdx.y;
    const int32_t group = i / N;
    const int64_t id = P[h * 4096 + i] - start;
    const int64_t anchor = (mode == 0 ? P[h * 4096 + group * N] : A[(h * 256 + group) * 2 + (mode - 1)]) - start;
    const float4* x = reinterpret_cast<const float4*>(U + ((int64_t)h * 4096 + id) * 128);
    const float4* y = reinterpret_cast<const float4*>(U + ((int64_t)h * 4096 + anchor) * 128);
    Acc4 acc;
#pragma unroll 8
    for (int w = 0; w < kWords; ++w) {
        const float4 a = x[w], b = y[w];
        acc.add((a.x * b.x), (a.y * b.y), (a.z * b.z), (a.w * b.w));
    }
    float value = acc.total();
    if (mode == 2) value = (value - S[h * 4096 + i]);
    S[h * 4096 + i] = value;
}

// Minimum of (ascending score key, position) words over a block.
__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int off) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, kWave);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, kWave);
    return ((uint64_t)hi << 32) | lo;
}

// fused_grouping.py:54-61: one 256-thread program per (group, head).
__global__ __launch_bounds__(256) void anchor_kernel(const int32_t* __restrict__ P, int32_t* A,
                                                     const float* __restrict__ S, const int32_t* flag, int32_t N,
                                                     int32_t slot) {
    __shared__ unsigned long long best;
    if (*flag >= 0) return;
    const int32_t group = blockIdx.x, h = blockIdx.y;
    if (threadIdx.x == 0) best = ~0ull;
    __syncthreads();
    uint64_t k = ~0ull;
    for (int32_t i = threadIdx.x; i < N; i += blockDim.x)
        k = umin64(k, ((uint64_t)score_key(S[h * 4096 + group * N + i]) << 32) | (uint32_t)i);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) k = umin64(k, shfl_xor64(k, off));
    if (__lane_id() == 0) atomicMin(&best, (unsigned long long)k);
    __syncthreads();
    if (threadIdx.x == 0) A[(h * 256 + group) * 2 + slot] = P[h * 4096 + group * N + (int32_t)(uint32_t)best];
}

// kernels.py:33-54: program (page, g) handles members g*8 .. g*8+7 of page,
// one thread per dim.
__global__ __launch_bounds__(128) void assemble_kernel(const uint8_t* __restrict__ K, const float* __restrict__ KS,
                                                       const int32_t* __restrict__ table, const int32_t* meta,
                                                       const int32_t* __restrict__ ids, uint8_t* tmp, float* tmps,
                                                       uint8_t* centers, float* cs, int32_t* map) {
    __shared__ float red[2];
    if (!meta[2]) return;
    const int32_t page = blockIdx.x, g = blockIdx.y, d = threadIdx.x;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int32_t i = g * 8 + j;
        const int32_t src = ids[page * 64 + i];
        const int64_t native = table[src / 64];
        const uint8_t code = K[native * V1_PAGE_BYTES + (src % 64) * 128 + d];
        const float scale = KS[native * kPageWords + kScaleWord + src % 64];
        tmp[(int64_t)page * V1_PAGE_BYTES + i * 128 + d] = code;
        if (d == 0) {
            tmps[(int64_t)page * kPageWords + kScaleWord + i] = scale;
            map[page * 64 + i] = meta[0] + src;
        }
        const float x = (__builtin_amdgcn_cvt_f32_fp8((int)code, 0) * scale);
        acc = j == 0 ? x : (acc + x);
    }
    const float mean = (acc * 0.125f);
    float amax = fabsf(mean);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    if (__lane_id() == 0) red[d / kWave] = amax;
    __syncthreads();
    const float scale = center_scale(fmaxf(red[0], red[1]));
    const int32_t c = page * 8 + g;
    centers[(int64_t)(c / 64) * V1_PAGE_BYTES + (c % 64) * 128 + d] = (uint8_t)e4m3_code(mean / scale);
    if (d == 0) cs[(int64_t)(c / 64) * kPageWords + kScaleWord + c % 64] = scale;
}

// ------------------------------------------------------------- fused
constexpr int kLevels = 7;  // groups of 1024, 512, ..., 16

struct BuildSmem {
    float4 anc[kTokens / 16][kWords];         // one anchor vector per group (<= 64 groups)
    unsigned long long rank_key[kTokens];     // (descending sort key, ~position) per position
    unsigned long long amin[2][kTokens / 16]; // argmin words per group, modes 0 and 1
    int32_t xtok[kTokens];                    // token at each new position
    float xf[kTokens];                        // and its unit factor
};
static_assert(sizeof(BuildSmem) <= 64 * 1024, "two work-groups per CU");

__global__ __launch_bounds__(kTokens) void build_buckets_kernel(const uint8_t* __restrict__ pool, int64_t pool_pages,
                                                                const int32_t* __restrict__ tables,
                                                                const int32_t* __restrict__ starts,
                                                                int32_t* __restrict__ perm_out,
                                                                uint8_t* __restrict__ tmp_out,
                                                                int32_t* __restrict__ map_out,
                                                                uint8_t* __restrict__ centers_out) {
    __shared__ BuildSmem sm;
    const int32_t p = threadIdx.x;  // position in the bucket's current order
    const int64_t b = blockIdx.x;
    const int32_t* table = tables + b * 16;
    const float* pool_f = reinterpret_cast<const float*>(pool);

    int32_t tok = p;
    uint32_t c[kWords];
    float s, f;
    auto fetch = [&]() __attribute__((always_inline)) {
        int64_t page = table[tok / 64];
        if ((uint64_t)page >= (uint64_t)pool_pages) page = 0;  // ids outside the pool read page 0
        load_key(pool + page * V1_PAGE_BYTES + (tok % 64) * 128, c);
        s = pool_f[page * kPageWords + kScaleWord + tok % 64];
    };
    fetch();
    f = unit_factor(c, s);

    // unit vector of this thread's token into anchor slot g
    auto put_anchor = [&](int32_t g) __attribute__((always_inline)) {
#pragma unroll
        for (int w = 0; w < kWords; ++w)
            sm.anc[g][w] = make_float4((fp8_at<0>(c[w]) * f), (fp8_at<1>(c[w]) * f),
                                       (fp8_at<2>(c[w]) * f), (fp8_at<3>(c[w]) * f));
    };
    auto dot = [&](int32_t g) __attribute__((always_inline)) {
        // the unit components are recomputed per dot: kept across the three
        // dots of a level they would need 128 more registers
#pragma unroll
        for (int w = 0; w < kWords; ++w) asm volatile("" : "+v"(c[w]));
        Acc4 acc;
#pragma unroll 4
        for (int w = 0; w < kWords; ++w) {
            const float4 a = sm.anc[g][w];
            acc.add(((fp8_at<0>(c[w]) * f) * a.x), ((fp8_at<1>(c[w]) * f) * a.y),
                    ((fp8_at<2>(c[w]) * f) * a.z), ((fp8_at<3>(c[w]) * f) * a.w));
        }
        return acc.total();
    };
    // group argmin (leftmost minimum, -0.0 == +0.0) into sm.amin[m][g]:
    // reduce over the wave's lanes of the group, then one atomic per wave
    auto argmin = [&](float v, int32_t n, int32_t g, int32_t m) __attribute__((always_inline)) {
        uint64_t k = ((uint64_t)score_key(v) << 32) | (uint32_t)p;
        const int width = n < kWave ? n : kWave;
        for (int off = 1; off < width; off <<= 1) k = umin64(k, shfl_xor64(k, off));
        if ((p & (width - 1)) == 0) atomicMin(&sm.amin[m][g], (unsigned long long)k);
    };

#pragma unroll 1
    for (int level = 0; level < kLevels; ++level) {
        const int32_t n = kTokens >> level;
        const int32_t g = p / n, gs = g * n;
        if (p == gs) {
            put_anchor(g);  // mode 0: the group's first member
            sm.amin[0][g] = ~0ull;
            sm.amin[1][g] = ~0ull;
        }
        __syncthreads();
        const float s0 = dot(g);
        argmin(s0, n, g, 0);
        __syncthreads();
        if (p == (int32_t)(uint32_t)sm.amin[0][g]) put_anchor(g);  // mode 1: b = argmin s0
        __syncthreads();
        const float sb = dot(g);
        argmin(sb, n, g, 1);
        __syncthreads();
        if (p == (int32_t)(uint32_t)sm.amin[1][g]) put_anchor(g);  // mode 2: a = argmin sb
        __syncthreads();
        const float score = (dot(g) - sb);
        // stable descending sort of the group: rank = members with a larger
        // (key, ~position) word
        const uint64_t key = ((uint64_t)score_key(score) << 32) | (0xffffffffu - (uint32_t)p);
        sm.rank_key[p] = key;
        __syncthreads();
        int32_t rank = 0;
        const ulonglong2* rk = reinterpret_cast<const ulonglong2*>(&sm.rank_key[gs]);
        for (int32_t q = 0; q < n / 2; ++q) {
            const ulonglong2 v = rk[q];
            rank += (v.x > key) + (v.y > key);
        }
        sm.xtok[gs + rank] = tok;
        sm.xf[gs + rank] = f;
        __syncthreads();
        tok = sm.xtok[p];
        f = sm.xf[p];
        fetch();
    }

    // final order: perm, the assembled pages, member map and centers
    perm_out[b * kTokens + p] = tok;
    map_out[b * kTokens + p] = starts[b] + tok;
    const int32_t page = p / 64, slot = p % 64;
    uint8_t* tp = tmp_out + (b * 16 + page) * V1_PAGE_BYTES;
    uint4* row = reinterpret_cast<uint4*>(tp + slot * 128);
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) row[i] = make_uint4(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
    reinterpret_cast<float*>(tp)[kScaleWord + slot] = s;
    // center p / 8: lane r of the 8 members computes dims 16r .. 16r+15 from
    // the members' key words 4r .. 4r+3 (lanes 8k .. 8k+7 of the wave)
    const int32_t r = p & 7, base = __lane_id() & ~7;
    float mean[16];
#pragma unroll 1
    for (int j = 0; j < 8; ++j) {
        const int src = base + j;
        const float sj = __shfl(s, src, kWave);
        uint32_t words[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // member j's word 4r+q: the word index depends on the reading
            // lane, so all eight candidates are shuffled and r picks one
            uint32_t w = 0;
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const uint32_t cand = (uint32_t)__shfl((int)c[4 * rr + q], src, kWave);
                w = r == rr ? cand : w;
            }
            words[q] = w;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x0 = (fp8_at<0>(words[q]) * sj), x1 = (fp8_at<1>(words[q]) * sj);
            const float x2 = (fp8_at<2>(words[q]) * sj), x3 = (fp8_at<3>(words[q]) * sj);
            if (j == 0) {
                mean[4 * q] = x0;
                mean[4 * q + 1] = x1;
                mean[4 * q + 2] = x2;
                mean[4 * q + 3] = x3;
            } else {
                mean[4 * q] = (mean[4 * q] + x0);
                mean[4 * q + 1] = (mean[4 * q + 1] + x1);
                mean[4 * q + 2] = (mean[4 * q + 2] + x2);
                mean[4 * q + 3] = (mean[4 * q + 3] + x3);
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        mean[i] = (mean[i] * 0.125f);
        amax = fmaxf(amax, fabsf(mean[i]));
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    const float scale = center_scale(amax);
    uint32_t packed[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        packed[q] = e4m3_code(mean[4 * q] / scale) | (e4m3_code(mean[4 * q + 1] / scale) << 8) |
                    (e4m3_code(mean[4 * q + 2] / scale) << 16) |
                    (e4m3_code(mean[4 * q + 3] / scale) << 24);
    const int32_t center = p / 8;
    uint8_t* cp = centers_out + (b * 2 + center / 64) * V1_PAGE_BYTES;
    *reinterpret_cast<uint4*>(cp + (center % 64) * 128 + 16 * r) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if (r == 0) reinterpret_cast<float*>(cp)[kScaleWord + center % 64] = scale;
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_build_initialize(const void* K, const float* KS, const int32_t* table, const int32_t* meta,
                                   float* unit, int32_t* perm, int32_t* flag, int32_t programs, void* stream) {
    V1_REQUIRE(programs >= 0, "initialize: negative grid");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(K) & 15) == 0 && (reinterpret_cast<uintptr_t>(unit) & 15) == 0,
               "initialize: K and UNIT must be 16-byte aligned");
    if (programs == 0) return V1_OK;
    hipLaunchKernelGGL(initialize_kernel, dim3((uint32_t)programs), dim3(64), 0, as_stream(stream),
                       static_cast<const uint8_t*>(K), KS, table, meta, unit, perm, flag);
    return V1_LAUNCHED("initialize");
}

extern "C" int v1_group_dots(const float* U, const int32_t* P, const int32_t* A, float* S, const int32_t* flag,
                             int32_t N, int32_t start, int32_t mode, int32_t programs, int32_t heads, void* stream) {
    V1_REQUIRE(N > 0 && mode >= 0 && mode <= 2 && programs >= 0 && heads >= 0, "_dots: bad arguments");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(U) & 15) == 0, "_dots: U must be 16-byte aligned");
    if (programs == 0 || heads == 0) return V1_OK;
    hipLaunchKernelGGL(dots_kernel, dim3((uint32_t)programs, (uint32_t)heads), dim3(64), 0, as_stream(stream), U, P, A,
                       S, flag, N, start, mode);
    return V1_LAUNCHED("_dots");
}

extern "C" int v1_group_anchor(const int32_t* P, int32_t* A, const float* S, const int32_t* flag, int32_t N,
                               int32_t slot, int32_t groups, int32_t heads, void* stream) {
    V1_REQUIRE(N > 0 && (slot == 0 || slot == 1) && groups >= 0 && heads >= 0, "_anchor: bad arguments");
    if (groups == 0 || heads == 0) return V1_OK;
    hipLaunchKernelGGL(anchor_kernel, dim3((uint32_t)groups, (uint32_t)heads), dim3(256), 0, as_stream(stream), P, A,
                       S, flag, N, slot);
    return V1_LAUNCHED("_anchor");
}

extern "C" int v1_build_assemble(const void* K, const float* KS, const int32_t* table, const int32_t* meta,
                                 const int32_t* ids, void* tmp, float* tmps, void* centers, float* cs, int32_t* map,
                                 int32_t pages, int32_t groups, void* stream) {
    V1_REQUIRE(pages >= 0 && groups >= 0 && groups <= 8, "assemble: bad grid");
    if (pages == 0 || groups == 0) return V1_OK;
    hipLaunchKernelGGL(assemble_kernel, dim3((uint32_t)pages, (uint32_t)groups), dim3(128), 0, as_stream(stream),
                       static_cast<const uint8_t*>(K), KS, table, meta, ids, static_cast<uint8_t*>(tmp), tmps,
                       static_cast<uint8_t*>(centers), cs, map);
    return V1_LAUNCHED("assemble");
}

extern "C" int v1_build_buckets(const void* pool, int64_t pool_pages, const int32_t* tables, const int32_t* starts,
                                int32_t buckets, int32_t* perm, void* tmp, int32_t* mapping, void* centers,
                                void* stream) {
    V1_REQUIRE(buckets >= 0 && pool_pages > 0, "build_buckets: bad shape");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(pool) & 15) == 0 && (reinterpret_cast<uintptr_t>(tmp) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(centers) & 15) == 0,
               "build_buckets: pool, tmp and centers must be 16-byte aligned");
    if (buckets == 0) return V1_OK;
    hipLaunchKernelGGL(build_buckets_kernel, dim3((uint32_t)buckets), dim3(kTokens), 0, as_stream(stream),
                       static_cast<const uint8_t*>(pool), pool_pages, tables, starts, perm, static_cast<uint8_t*>(tmp), mapping,
                       static_cast<uint8_t*>(centers));
    return V1_LAUNCHED("build_buckets");
}
