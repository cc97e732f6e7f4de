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
// follow kernels.py:17-28: x_d = fl(c_d * s), m = max(sqrt(sum x_d^2), 1e-12),
// u_d = fl(x_d / m), c_d the FP8 key and s its scale.  Center means add the 8
// members in order, times 1/8.
//
// Two forms: per-kernel drop-ins with the reference's launch shapes, and one
// fused kernel that builds a batch of buckets, one 1024-thread work-group per
// bucket (thread = position in the bucket's order): the token's FP8 key stays
// in registers, an argmin winner stages its key in LDS for the lanes that
// expand the anchor, each group is sorted by a bitonic network over its
// unique (score, -position) words, and members move through LDS (groups
// larger than a wave) or lane shuffles.
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

// Divisor m of a token's unit vector: max(||x||, 1e-12), x_d = c_d * s.
__device__ __forceinline__ float unit_norm(const uint32_t (&c)[kWords], float s) {
    Acc4 acc;
#pragma unroll
    for (int w = 0; w < kWords; ++w) {
        const float x0 = (fp8_at<0>(c[w]) * s), x1 = (fp8_at<1>(c[w]) * s);
        const float x2 = (fp8_at<2>(c[w]) * s), x3 = (fp8_at<3>(c[w]) * s);
        acc.add((x0 * x0), (x1 * x1), (x2 * x2), (x3 * x3));
    }
    return fmaxf(sqrtf(acc.total()), 1e-12f);
}

// fl(x / m) from r = fl(1 / m): q0 = fl(x * r), then one correction with the
// exact residual x - q0 * m (an FMA).  With a correctly rounded reciprocal the
// corrected quotient is the correctly rounded one (Markstein's division
// theorem; checked against the division on 3.9e8 x = fp8 * s, m >= |x| pairs,
// significands of m all ones and near powers of two included).  x = -0 gives
// +0 where the division gives -0: the dots cannot tell, every partial sum
// starts at +0.
__device__ __forceinline__ float unit_div(float x, float m, float r) {
    const float q0 = x * r;
    return __builtin_fmaf(__builtin_fmaf(-q0, m, x), r, q0);
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
    const float m = unit_norm(c, s);
    float4* dst = reinterpret_cast<float4*>(unit + (int64_t)i * 128);
#pragma unroll
    for (int w = 0; w < kWords; ++w)
        dst[w] = make_float4((fp8_at<0>(c[w]) * s) / m, (fp8_at<1>(c[w]) * s) / m,
                             (fp8_at<2>(c[w]) * s) / m, (fp8_at<3>(c[w]) * s) / m);
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
constexpr int kLevels = 7;      // groups of 1024, 512, ..., 16
constexpr int kSlots = 64;      // anchor and stage slots: four per wave
constexpr int kAncStride = 33;  // float4 per anchor slot, one of padding

// A token's FP8 key, scale and unit divisor, staged for the lanes that expand it.
struct Stage {
    uint32_t c[kWords];
    float s, m;
    uint32_t pad[2];
};

struct BuildSmem {
    union {
        struct {
            float4 anc[kSlots][kAncStride];  // anchor unit vectors: one per wave (groups >= 64) or group
            Stage st[2][kSlots];             // argmin winners of the first and second dot
        } d;                                 // live from a level's first anchor to its last dot
        struct {
            uint2 c[kWords / 2][kTokens];    // keys by position, 8 bytes of every row per plane
            int32_t tok[kTokens];
            float s[kTokens];                // scales
            float m[kTokens];                // unit divisors
        } x;                                 // live during a block-wide exchange and the final assembly
    } u1;
    union {
        unsigned long long k[2][kTokens];    // sort keys crossing waves, double-buffered
        Stage st0[kSlots];                   // first members of the next level's groups
    } u2;
    unsigned long long amin[2][kSlots];      // group argmin words (groups above one wave)
};
static_assert(sizeof(BuildSmem) <= 160 * 1024, "one work-group per CU");

// Orders this wave's LDS accesses across its lanes (a wave's LDS operations
// complete in order; the wait and the empty barrier keep the compiler from
// moving accesses across the point).
__device__ __forceinline__ void wave_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// FP8 bytes 2H and 2H+1 of a packed word, as fp32 (exact).
template <bool H>
__device__ __forceinline__ float2 fp8_pair(uint32_t w) {
    const auto v = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, H);
    return make_float2(v[0], v[1]);
}

// Lane p ^ J's value (J < 64, every lane active): DPP quad permutes and a
// row rotate for 1, 2 and 8, swizzle bit masks for 4 and 16, a permute for 32.
template <int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    if constexpr (J == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (J == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (J == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);
    else if constexpr (J == 4 || J == 16) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (J << 10) | 0x1F);
    else return (uint32_t)__shfl_xor((int)v, J, kWave);
}

template <int J>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
    return ((uint64_t)lane_xor<J>((uint32_t)(v >> 32)) << 32) | lane_xor<J>((uint32_t)v);
}

// One compare-exchange step of a descending bitonic network over groups of
// N (i = position in the group, partner i ^ J, merge size S).
template <int N, int S, int J>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t key, int32_t p, uint64_t (*buf)[kTokens], int32_t& nb) {
    uint64_t other;
    if constexpr (J >= kWave) {
        buf[nb][p] = key;
        __syncthreads();
        other = buf[nb][p ^ J];
        nb ^= 1;
    } else {
        other = lane_xor64<J>(key);
    }
    const int32_t i = p & (N - 1);
    const bool take_max = ((i & J) == 0) == ((i & S) == 0);
    // keys of a group are distinct, so one compare decides: keep the partner's
    // key when it is the larger and this position keeps the maximum, or the
    // smaller and it keeps the minimum
    const bool other_gt = other > key;
    return other_gt == take_max ? other : key;
}

template <int N, int S, int J>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t key, int32_t p, uint64_t (*buf)[kTokens], int32_t& nb) {
    key = bitonic_step<N, S, J>(key, p, buf, nb);
    if constexpr (J > 1) key = bitonic_merge<N, S, J / 2>(key, p, buf, nb);
    return key;
}

// Descending sort of every aligned group of N keys (unique); strides of a
// wave or more exchange through buf (double-buffered, barriers between).
template <int N, int S = 2>
__device__ __forceinline__ uint64_t bitonic_sort(uint64_t key, int32_t p, uint64_t (*buf)[kTokens], int32_t& nb) {
    key = bitonic_merge<N, S, S / 2>(key, p, buf, nb);
    if constexpr (S < N) key = bitonic_sort<N, S * 2>(key, p, buf, nb);
    return key;
}

// One 1024-thread work-group per bucket; thread = position in the bucket's
// current order.  Per level (groups of n): three dots against the group's
// anchors (first member, b = argmin s0, a = argmin sb), score = dot_a - sb,
// and a stable descending sort of every group by (score, -position).
// Groups of at most one wave run without block barriers; larger groups
// reduce their argmin through LDS atomics and exchange members through LDS.
__global__ __launch_bounds__(kTokens) void build_buckets_kernel(const uint8_t* __restrict__ pool, int64_t pool_pages,
                                                                const int32_t* __restrict__ tables,
                                                                const int32_t* __restrict__ starts,
                                                                int32_t* __restrict__ perm_out,
                                                                uint8_t* __restrict__ tmp_out,
                                                                int32_t* __restrict__ map_out,
                                                                uint8_t* __restrict__ centers_out) {
    __shared__ BuildSmem sm;
    const int32_t p = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int32_t* table = tables + b * 16;
    const float* pool_f = reinterpret_cast<const float*>(pool);
    auto page_of = [&](int32_t t) __attribute__((always_inline)) {
        int64_t page = table[t / 64];
        if ((uint64_t)page >= (uint64_t)pool_pages) page = 0;  // ids outside the pool read page 0
        return page;
    };

    int32_t tok = p;
    uint32_t c[kWords];
    float s, m, rm;  // the token's scale, unit divisor and its reciprocal
    {
        const int64_t page = page_of(tok);
        load_key(pool + page * V1_PAGE_BYTES + (tok % 64) * 128, c);
        s = pool_f[page * kPageWords + kScaleWord + tok % 64];
        m = unit_norm(c, s);
        rm = 1.0f / m;
    }

    // slot of position q's group within q's wave (groups of `width` <= 64
    // lanes): every wave owns slots 4w .. 4w+3 at every level, so levels run
    // without block barriers never touch another wave's slots
    auto wslot = [](int32_t q, int32_t width) __attribute__((always_inline)) {
        return (q >> 6) * 4 + (q & (kWave - 1)) / width;
    };
    auto stage_put = [&](Stage& st) __attribute__((always_inline)) {
        uint4* dst = reinterpret_cast<uint4*>(st.c);
#pragma unroll
        for (int i = 0; i < kWords / 4; ++i) dst[i] = make_uint4(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
        st.s = s;
        st.m = m;
    };
    // anchor slot `slot` <- unit vector of the staged token; the `width`
    // lanes sharing the slot expand one or two key words each
    auto expand = [&](const Stage& st, int32_t slot, int32_t width) __attribute__((always_inline)) {
        const int32_t j = p & (width - 1);
        const int32_t per = width >= 32 ? 1 : 32 / width;  // 1 or 2 (width >= 16)
        if (j * per < kWords) {
            const float sa = st.s, ma = st.m;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (q < per) {
                    const int32_t w = j * per + q;
                    const uint32_t cw = st.c[w];
                    const float2 lo = fp8_pair<false>(cw), hi = fp8_pair<true>(cw);
                    sm.u1.d.anc[slot][w] =
                        make_float4((lo.x * sa) / ma, (lo.y * sa) / ma, (hi.x * sa) / ma, (hi.y * sa) / ma);
                }
            }
        }
    };
    auto dot = [&](int32_t slot) __attribute__((always_inline)) {
        // the unit components are recomputed per dot: kept across the three
        // dots of a level they would need 128 more registers
#pragma unroll
        for (int w = 0; w < kWords; ++w) asm volatile("" : "+v"(c[w]));
        const float4* a = sm.u1.d.anc[slot];
        Acc4 acc;
#pragma unroll 4
        for (int w = 0; w < kWords; ++w) {
            const float4 av = a[w];
            const float2 lo = fp8_pair<false>(c[w]), hi = fp8_pair<true>(c[w]);
            acc.add((unit_div(lo.x * s, m, rm) * av.x), (unit_div(lo.y * s, m, rm) * av.y),
                    (unit_div(hi.x * s, m, rm) * av.z), (unit_div(hi.y * s, m, rm) * av.w));
        }
        return acc.total();
    };
    // group argmin (leftmost minimum, -0.0 == +0.0): the winner stages its
    // key in st[m][its slot]; returns the winner's position
    auto argmin = [&](float v, int32_t n, int32_t width, int32_t m) __attribute__((always_inline)) {
        uint64_t k = ((uint64_t)score_key(v) << 32) | (uint32_t)p;
        k = umin64(k, lane_xor64<1>(k));  // width >= 16
        k = umin64(k, lane_xor64<2>(k));
        k = umin64(k, lane_xor64<4>(k));
        k = umin64(k, lane_xor64<8>(k));
        if (width > 16) k = umin64(k, lane_xor64<16>(k));
        if (width > 32) k = umin64(k, lane_xor64<32>(k));
        if ((uint32_t)k == (uint32_t)p) stage_put(sm.u1.d.st[m][wslot(p, width)]);
        if (n > kWave) {
            if ((p & (kWave - 1)) == 0) atomicMin(&sm.amin[m][p / n], (unsigned long long)k);
            __syncthreads();
            k = sm.amin[m][p / n];
        } else {
            wave_sync();
        }
        return (int32_t)(uint32_t)k;
    };
    if (p < 2 * kSlots) (&sm.amin[0][0])[p] = ~0ull;
    if (p == 0) stage_put(sm.u2.st0[0]);
    __syncthreads();

#pragma unroll 1
    for (int level = 0; level < kLevels; ++level) {
        const int32_t n = kTokens >> level;
        const int32_t width = n < kWave ? n : kWave;
        const int32_t slot = wslot(p, width);
        expand(sm.u2.st0[n > kWave ? p / n : slot], slot, width);  // the group's first member
        wave_sync();
        const float s0 = dot(slot);
        const int32_t bpos = argmin(s0, n, width, 0);
        expand(sm.u1.d.st[0][wslot(bpos, width)], slot, width);
        wave_sync();
        const float sb = dot(slot);
        const int32_t apos = argmin(sb, n, width, 1);
        expand(sm.u1.d.st[1][wslot(apos, width)], slot, width);
        wave_sync();
        const float score = (dot(slot) - sb);
        uint64_t key = ((uint64_t)score_key(score) << 32) | (0xffffffffu - (uint32_t)p);
        {
            auto* kb = reinterpret_cast<uint64_t (*)[kTokens]>(sm.u2.k);
            int32_t nb = 0;
            switch (level) {
                case 0: key = bitonic_sort<1024>(key, p, kb, nb); break;
                case 1: key = bitonic_sort<512>(key, p, kb, nb); break;
                case 2: key = bitonic_sort<256>(key, p, kb, nb); break;
                case 3: key = bitonic_sort<128>(key, p, kb, nb); break;
                case 4: key = bitonic_sort<64>(key, p, kb, nb); break;
                case 5: key = bitonic_sort<32>(key, p, kb, nb); break;
                default: key = bitonic_sort<16>(key, p, kb, nb); break;
            }
        }
        const int32_t from = (int32_t)(0xffffffffu - (uint32_t)key);  // old position of the new member
        const int32_t half = n >> 1;
        if (n > kWave) {
            // every wave is past its last dot (the sort crossed a barrier):
            // the exchange area may overwrite the anchors
#pragma unroll
            for (int w = 0; w < kWords / 2; ++w) sm.u1.x.c[w][p] = make_uint2(c[2 * w], c[2 * w + 1]);
            sm.u1.x.tok[p] = tok;
            sm.u1.x.s[p] = s;
            sm.u1.x.m[p] = m;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < kWords / 2; ++w) {
                const uint2 v = sm.u1.x.c[w][from];
                c[2 * w] = v.x;
                c[2 * w + 1] = v.y;
            }
            tok = sm.u1.x.tok[from];
            s = sm.u1.x.s[from];
            m = sm.u1.x.m[from];
            rm = 1.0f / m;
            if (p < 2 * kSlots) (&sm.amin[0][0])[p] = ~0ull;
            if (level + 1 < kLevels && (p & (half - 1)) == 0)
                stage_put(sm.u2.st0[half > kWave ? p / half : wslot(p, half)]);
            __syncthreads();
        } else {
            const int32_t src = from & (kWave - 1);  // same wave
#pragma unroll
            for (int w = 0; w < kWords; ++w) c[w] = (uint32_t)__shfl((int)c[w], src, kWave);
            tok = __shfl(tok, src, kWave);
            s = __shfl(s, src, kWave);
            m = __shfl(m, src, kWave);
            rm = __shfl(rm, src, kWave);
            if (level + 1 < kLevels && (p & (half - 1)) == 0) stage_put(sm.u2.st0[wslot(p, half)]);
            wave_sync();
        }
    }

    // final order: perm, the assembled pages, member map and centers
    const int64_t page = page_of(tok);
    perm_out[b * kTokens + p] = tok;
    map_out[b * kTokens + p] = starts[b] + tok;
    uint8_t* tp = tmp_out + (b * 16 + p / 64) * V1_PAGE_BYTES;
    uint4* row = reinterpret_cast<uint4*>(tp + (p % 64) * 128);
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) row[i] = make_uint4(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
    reinterpret_cast<float*>(tp)[kScaleWord + p % 64] = s;
    __syncthreads();  // every wave is past its last dot
#pragma unroll
    for (int w = 0; w < kWords / 2; ++w) sm.u1.x.c[w][p] = make_uint2(c[2 * w], c[2 * w + 1]);
    sm.u1.x.s[p] = s;
    wave_sync();  // a center's 8 members are rows of this wave
    // center p / 8: lane r of the 8 members computes dims 16r .. 16r+15
    const int32_t r = p & 7, m0 = p & ~7;
    float mean[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint2 w01 = sm.u1.x.c[2 * r][m0 + j], w23 = sm.u1.x.c[2 * r + 1][m0 + j];
        const float sj = sm.u1.x.s[m0 + j];
        const uint32_t words[4] = {w01.x, w01.y, w23.x, w23.y};
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
