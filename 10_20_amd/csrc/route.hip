// fused.route (page max-of-8 + stable top-`take` page selection + fine page
// table) and the _sort group sort.  Both order a small set (<= 4096) by
// "value descending, then index ascending", which is a strict total order on
// the 64-bit composite (order-preserving value key << 32) | ~index.  A bitonic
// network over that composite in LDS is therefore deterministic and stable by
// construction; one work-group sorts one route row or several _sort groups.
#include "common.h"

namespace v1 {
namespace {

constexpr int kMaxSort = 4096;

// Bitonic sort of s[0..n) descending, where n is a power of two and every
// aligned run of `group` elements is sorted independently (group divides n).
template <typename Less>
__device__ void bitonic_desc(uint64_t* s, int n, int group, Less less) {
    for (int k = 2; k <= group; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (j - 1));
                const int hi = lo + j;
                const bool desc = k == group ? true : ((lo & k) == 0);
                const uint64_t a = s[lo], b = s[hi];
                if (desc ? less(a, b) : less(b, a)) {
                    s[lo] = b;
                    s[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

struct U64Less {
    __device__ bool operator()(uint64_t a, uint64_t b) const { return a < b; }
};

// sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:7-49
template <typename Index, int E>
__global__ __launch_bounds__(512) void route_kernel(v1_route_args a, int n_sort) {
    __shared__ uint64_t s0[512 * E], s1[512 * E];  // (E = n_sort / 512: 8 KB of LDS per 512 keys)
    const int64_t row = blockIdx.x;
    const int32_t active = max(a.lens[row] - 1, 0) / 1024 * 16;
    const int32_t take = a.takes[row];
    Index* selected = static_cast<Index*>(a.selected) + row * a.take_stride;
    int32_t* ft = a.ft + row * a.ft_cols;
    const int32_t* rt = a.rt + row * a.pages;
    if (a.fill_table)
        for (int j = max(take, 0) + threadIdx.x; j < a.ft_cols; j += blockDim.x)
            ft[j] = a.capacity + a.tail_rows[row] * 68 + min(j - take, 67);
    if (take >= active) {
        for (int i = threadIdx.x; i < a.take_stride; i += blockDim.x) {
            selected[i] = (Index)i;
            if (a.fill_table && i < take && i < a.pages) ft[i] = rt[i];
        }
        return;
    }
    const float* sc = a.scores + row * a.score_stride;
    const int e0 = (int)threadIdx.x * E;
    uint64_t v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int p = e0 + i;
        v[i] = 0;  // padding slots sort last
        if (p < a.pages) {
            float best = -__builtin_huge_valf();
            if (p < active) {
                const float4 x = reinterpret_cast<const float4*>(sc + 8 * p)[0];
                const float4 y = reinterpret_cast<const float4*>(sc + 8 * p)[1];
                best = fmaxf(fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)), fmaxf(fmaxf(y.x, y.y), fmaxf(y.z, y.w)));
            }
            v[i] = ((uint64_t)score_key(best) << 32) | (uint32_t)(0xffffffffu - (uint32_t)p);
        }
    }
    // Only the first n = pow2(active) slots are sorted: every slot past them
    // holds a page at or past `active` (a -inf score) or padding, which the
    // whole sort would leave in place (-inf pages in ascending order after
    // every active page), so rank r >= n is page r.  (The network's steps
    // pair slots below n only with each other.)
    const int n = min(n_sort, active <= 2 ? 2 : 1 << (32 - __builtin_clz((uint32_t)(active - 1))));
    bitonic_desc_regs<E>(v, n, s0, s1, n);
    // selected takes ranks < take_stride; the fine table every rank < take
    // (v1_query.cuh:44-48), bounded by the sorted pages and the table width
    const int32_t ft_ranks = a.fill_table ? min(min(take, a.pages), a.ft_cols) : 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int r = e0 + i;
        const int32_t p = r < n ? (int32_t)(0xffffffffu - (uint32_t)v[i]) : r;
        if (r < a.take_stride) selected[r] = (Index)p;
        if (r < ft_ranks) ft[r] = rt[p];
    }
}

// sglang/srt/layers/attention/v1_native/fused_grouping.py:64-76.  Block b,
// head h sorts groups [b*gpb, (b+1)*gpb) of head h.
__global__ __launch_bounds__(256) void sort_f32_kernel(const int32_t* perm, int32_t* out, const float* keys,
                                                       const int32_t* flag, int32_t n, int32_t groups,
                                                       int32_t gpb, int64_t head_stride) {
    __shared__ uint64_t s[kMaxSort];
    if (*flag >= 0) return;
    const int64_t h = blockIdx.y;
    const int32_t g0 = blockIdx.x * gpb;
    const int32_t ng = min(gpb, groups - g0);
    const int m = ng * n;
    const int64_t base = h * head_stride + (int64_t)g0 * n;
    for (int i = threadIdx.x; i < m; i += blockDim.x) {
        const uint32_t pos = (uint32_t)(i % n);
        s[i] = ((uint64_t)score_key(keys[base + i]) << 32) | (0xffffffffu - pos);
    }
    __syncthreads();
    bitonic_desc(s, m, n, U64Less{});
    for (int i = threadIdx.x; i < m; i += blockDim.x) {
        const int32_t g = i / n;
        const int32_t pos = (int32_t)(0xffffffffu - (uint32_t)s[i]);
        out[base + i] = perm[base + (int64_t)g * n + pos];
    }
}

// sort_f32_kernel for groups of at most 1024 (the reference's sizes): the
// block's 1024 slots are held four per thread in registers, so only the steps
// that pair elements of different waves (j >= 256) go through LDS.
__global__ __launch_bounds__(256) void sort_f32_regs_kernel(const int32_t* perm, int32_t* out, const float* keys,
                                                            const int32_t* flag, int32_t n, int32_t groups,
                                                            int32_t gpb, int64_t head_stride) {
    constexpr int E = 4;
    __shared__ uint64_t s0[256 * E], s1[256 * E];
    if (*flag >= 0) return;
    const int64_t h = blockIdx.y;
    const int32_t g0 = blockIdx.x * gpb;
    const int32_t ng = min(gpb, groups - g0);
    const int m = ng * n;
    const int64_t base = h * head_stride + (int64_t)g0 * n;
    const int e0 = (int)threadIdx.x * E;
    uint64_t v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int p = e0 + i;
        v[i] = p < m ? ((uint64_t)score_key(keys[base + p]) << 32) | (0xffffffffu - (uint32_t)(p % n)) : 0ull;
    }
    // (slots past m form whole groups of their own: they never mix with real ones)
    bitonic_desc_regs<E>(v, 256 * E, s0, s1, n);
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int p = e0 + i;
        if (p < m) out[base + p] = perm[base + (int64_t)(p / n) * n + (int32_t)(0xffffffffu - (uint32_t)v[i])];
    }
}

// Same rule over signed 64-bit keys: the composite does not fit 64 bits, so
// the network carries indices and compares (key desc, position asc).
__global__ __launch_bounds__(256) void sort_i64_kernel(const int32_t* perm, int32_t* out, const int64_t* keys,
                                                       const int32_t* flag, int32_t n, int32_t groups, int32_t gpb) {
    __shared__ uint64_t s[kMaxSort];  // low 32 bits: element index inside the block
    __shared__ int64_t k[kMaxSort];
    if (flag != nullptr && *flag >= 0) return;
    const int32_t g0 = blockIdx.x * gpb;
    const int32_t ng = min(gpb, groups - g0);
    const int m = ng * n;
    const int64_t base = (int64_t)g0 * n;
    for (int i = threadIdx.x; i < m; i += blockDim.x) {
        s[i] = (uint64_t)i;
        k[i] = keys[base + i];
    }
    __syncthreads();
    // a "less" b  <=>  a comes after b in the descending stable order
    auto less = [&](uint64_t a, uint64_t b) {
        const int64_t ka = k[(int)a], kb = k[(int)b];
        return ka < kb || (ka == kb && a > b);
    };
    bitonic_desc(s, m, n, less);
    for (int i = threadIdx.x; i < m; i += blockDim.x) out[base + i] = perm[base + (int64_t)s[i]];
}

int pow2_at_least(int x) {
    int n = 1;
    while (n < x) n <<= 1;
    return n;
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_route(const v1_route_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "route: null args");
    V1_REQUIRE(a->capacity > 0 && a->ft_cols >= a->take_stride, "Invalid fine page table");
    V1_REQUIRE(a->pages >= 64 && a->pages <= 4096 && a->score_cols >= a->pages * 8 &&
                   a->take_stride <= a->pages && a->score_stride % 4 == 0,
               "Invalid V1 route capacity");
    V1_REQUIRE(a->selected_bits == 32 || a->selected_bits == 64, "route: selected must be int32 or int64");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(a->scores) & 15) == 0, "route: scores must be 16-byte aligned");
    if (a->batch == 0) return V1_OK;
    const int n_sort = pow2_at_least(a->pages);  // 64 .. 4096: E = n_sort / 512 keys per thread, at least 1
    hipStream_t st = as_stream(stream);
    const dim3 g(a->batch), b(512);
    if (a->selected_bits == 32) {
        if (n_sort <= 512) hipLaunchKernelGGL((route_kernel<int32_t, 1>), g, b, 0, st, *a, n_sort);
        else if (n_sort == 1024) hipLaunchKernelGGL((route_kernel<int32_t, 2>), g, b, 0, st, *a, n_sort);
        else if (n_sort == 2048) hipLaunchKernelGGL((route_kernel<int32_t, 4>), g, b, 0, st, *a, n_sort);
        else hipLaunchKernelGGL((route_kernel<int32_t, 8>), g, b, 0, st, *a, n_sort);
    } else {
        if (n_sort <= 512) hipLaunchKernelGGL((route_kernel<int64_t, 1>), g, b, 0, st, *a, n_sort);
        else if (n_sort == 1024) hipLaunchKernelGGL((route_kernel<int64_t, 2>), g, b, 0, st, *a, n_sort);
        else if (n_sort == 2048) hipLaunchKernelGGL((route_kernel<int64_t, 4>), g, b, 0, st, *a, n_sort);
        else hipLaunchKernelGGL((route_kernel<int64_t, 8>), g, b, 0, st, *a, n_sort);
    }
    return V1_LAUNCHED("route");
}

extern "C" int v1_sort_f32(const int32_t* perm, int32_t* out, const float* keys, const int32_t* flag, int32_t n,
                           int32_t groups, int32_t heads, int64_t head_stride, void* stream) {
    V1_REQUIRE(n >= 2 && n <= kMaxSort && (n & (n - 1)) == 0, "sort: group size must be a power of two in [2, 4096]");
    V1_REQUIRE(groups >= 0 && heads >= 0, "sort: bad shape");
    V1_REQUIRE(perm != out, "P and O must be distinct non-overlapping buffers");
    V1_REQUIRE(flag != nullptr, "sort: flag required");
    if (groups == 0 || heads == 0) return V1_OK;
    const int gpb = max(1, min(groups, 1024 / n));
    if (n <= 1024)
        hipLaunchKernelGGL(sort_f32_regs_kernel, dim3((uint32_t)cdiv(groups, gpb), heads), dim3(256), 0,
                           as_stream(stream), perm, out, keys, flag, n, groups, gpb, head_stride);
    else
        hipLaunchKernelGGL(sort_f32_kernel, dim3((uint32_t)cdiv(groups, gpb), heads), dim3(256), 0, as_stream(stream),
                           perm, out, keys, flag, n, groups, gpb, head_stride);
    return V1_LAUNCHED("sort_f32");
}

extern "C" int v1_sort_i64(const int32_t* perm, int32_t* out, const int64_t* keys, const int32_t* flag, int32_t n,
                           int32_t groups, void* stream) {
    V1_REQUIRE(n >= 2 && n <= kMaxSort && (n & (n - 1)) == 0, "sort: group size must be a power of two in [2, 4096]");
    V1_REQUIRE(groups >= 0, "sort: bad shape");
    V1_REQUIRE(perm != out, "P and O must be distinct non-overlapping buffers");
    if (groups == 0) return V1_OK;
    const int gpb = max(1, min(groups, 1024 / n));
    hipLaunchKernelGGL(sort_i64_kernel, dim3((uint32_t)cdiv(groups, gpb)), dim3(256), 0, as_stream(stream), perm,
                       out, keys, flag, n, groups, gpb);
    return V1_LAUNCHED("sort_i64");
}
