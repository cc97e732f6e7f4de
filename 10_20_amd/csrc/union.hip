// Shared sink + tail staging for one request's causal chunk, and the page
// tables, score normalisation and Top-K mapping around it.
//
// Semantics: experiments/tail_union_lab_20261021/union.py:10-42 (bounds,
// stage_union), experiments/fine_pool_shared_20261021/kernels.py:7-76
// (tables, normalize, map_topk).  Every query row r of the chunk (lengths
// lens[r], non-negative and non-decreasing) scores the candidates
//   sink [0, s) + tail [t, n),   s = min(n, S),
//   t = max(s, min(min(max(end, 0), n), max(s, n - W))),  count = s + n - t,
// where `end` (indexed_end) is the end of the contiguous prefix whose index
// is published: every visible token at or past it is a tail candidate.
// Instead of one staged copy per row, the union of all rows' candidate pages
// (sink pages [0, sp) and tail pages [tp, ep)) is copied once into the fine
// pool; each row's page table points into that union, and `normalize`
// restores the scores to the canonical candidate order (history pages, sink,
// tail) the Top-K and `map_topk` expect.
//
// Deviations (inputs the reference leaves undefined): page ids outside the
// source pool or the page table stage zero pages; selected / member entries
// outside their arrays, and logical positions past the page table, make a
// candidate invalid (-inf, id -1) instead of reading past the buffer.
#include "common.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace v1 {
namespace {

struct UnionBounds {
    int32_t s, t, c;
};

// union.py:10-14
__device__ __forceinline__ UnionBounds union_bounds(int32_t n, int32_t end, int32_t S, int32_t W) {
    const int32_t s = min(n, S);
    const int32_t t = max(s, min(min(max(end, 0), n), max(s, n - W)));
    return {s, t, s + n - t};
}

// The union's page ranges from the first and last rows (union.py:18-24).
struct UnionPages {
    int32_t sp, tp, ep, total;
};

__device__ __forceinline__ UnionPages union_pages(const int32_t* lens, int32_t rows, int32_t end, int32_t S,
                                                  int32_t W) {
    const int32_t first = lens[0], last = lens[rows - 1];
    UnionPages u;
    u.sp = (min(last, S) + 63) / 64;
    u.tp = max(u.sp, union_bounds(first, end, S, W).t / 64);
    u.ep = (last + 63) / 64;
    u.total = u.sp + max(u.ep - u.tp, 0);
    return u;
}

// Blocks [0, dst_pages): union page b <- source page nt[b < sp ? b : tp + b - sp]
// (pages past the union are left alone); the next blocks write each row's
// (s, t, count) and the first of them the descriptor (sp, tp, ep, total).
__global__ __launch_bounds__(256) void stage_union_kernel(const uint8_t* __restrict__ src, int64_t src_pages,
                                                          const int32_t* __restrict__ nt, int32_t nt_len,
                                                          const int32_t* __restrict__ lens, int32_t rows,
                                                          const int32_t* __restrict__ indexed_end,
                                                          uint8_t* __restrict__ dst, int32_t dst_pages,
                                                          int32_t* __restrict__ meta, int32_t* __restrict__ desc,
                                                          int32_t S, int32_t W) {
    const int32_t end = *indexed_end;
    const UnionPages u = union_pages(lens, rows, end, S, W);
    const int32_t b = blockIdx.x;
    if (b < dst_pages) {
        if (b >= u.total) return;
        const int32_t lp = b < u.sp ? b : u.tp + b - u.sp;
        const int64_t page = (lp >= 0 && lp < nt_len) ? nt[lp] : -1;
        const bool ok = page >= 0 && page < src_pages;
        const u32x4* in = reinterpret_cast<const u32x4*>(src + (ok ? page : 0) * V1_PAGE_BYTES);
        u32x4* out = reinterpret_cast<u32x4*>(dst + (int64_t)b * V1_PAGE_BYTES);
        for (int c = threadIdx.x; c < V1_PAGE_BYTES / 16; c += 256) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (ok) v = in[c];
            out[c] = v;
        }
        return;
    }
    const int32_t mb = b - dst_pages;
    if (mb == 0 && threadIdx.x == 0) {
        desc[0] = u.sp;
        desc[1] = u.tp;
        desc[2] = u.ep;
        desc[3] = u.total;
    }
    const int32_t r = mb * 256 + threadIdx.x;
    if (r < rows) {
        const UnionBounds x = union_bounds(lens[r], end, S, W);
        meta[3 * r] = x.s;
        meta[3 * r + 1] = x.t;
        meta[3 * r + 2] = x.c;
    }
}

// kernels.py:13-35: row r's fine table (history pages, then its sink and
// tail pages: in the union when shared, in its own scratch pages otherwise),
// the span DeepGEMM scores and the canonical candidate count.
__global__ __launch_bounds__(256) void union_tables_kernel(const int32_t* __restrict__ lens,
                                                           const int32_t* __restrict__ indexed_end,
                                                           const int32_t* __restrict__ takes,
                                                           const int32_t* __restrict__ selected,
                                                           const int32_t* __restrict__ desc, int32_t* __restrict__ ft,
                                                           int32_t* __restrict__ dg_lens, int32_t* __restrict__ clens,
                                                           int32_t cap, int32_t max_take, int32_t scratch, int32_t fp,
                                                           int32_t S, int32_t W, int32_t shared) {
    const int64_t r = blockIdx.x;
    const int32_t n = lens[r], take = takes[r];
    const UnionBounds x = union_bounds(n, *indexed_end, S, W);
    int32_t pages, span, sp = 0, tp = 0, gsp = 0, gtp = 0;
    if (shared) {
        sp = (x.s + 63) / 64;
        tp = max(sp, x.t / 64);
        const int32_t ep = (n + 63) / 64;
        gsp = desc[0];
        gtp = desc[1];
        pages = sp + max(ep - tp, 0);
        span = ep > tp ? sp * 64 + n - tp * 64 : n;
    } else {
        pages = (x.c + 63) / 64;
        span = x.c;
    }
    for (int32_t j = threadIdx.x; j < fp; j += 256) {
        int32_t v;
        if (j < take) {
            v = j < max_take ? selected[r * max_take + j] : 0;
        } else {
            const int32_t k = j - take;
            const int32_t page = shared ? (k < sp ? cap + k : cap + gsp + tp - gtp + k - sp)
                                        : cap + (int32_t)r * scratch + k;
            v = (k >= 0 && k < pages) ? page : 0;
        }
        ft[r * fp + j] = v;
    }
    if (threadIdx.x == 0) {
        dg_lens[r] = max(take * 64 + span, 1);
        clens[r] = take * 64 + x.c;
    }
}

// kernels.py:38-59: canonical candidate j of row r (history member, sink,
// tail) <- its raw score (shared: the tail's place in the union's span),
// -inf where the member is outside [s, t) or past n / end, or j >= count.
// Four consecutive candidates per thread (one 16-byte store when the row
// allows it).
__global__ __launch_bounds__(256) void union_normalize_kernel(const float* __restrict__ raw, int64_t raw_stride,
                                                              int32_t raw_cols, const int32_t* __restrict__ lens,
                                                              const int32_t* __restrict__ indexed_end,
                                                              const int32_t* __restrict__ takes,
                                                              const int32_t* __restrict__ selected,
                                                              const int32_t* __restrict__ members,
                                                              int64_t members_pages, float* __restrict__ out,
                                                              int32_t max_take, int32_t width, int32_t S, int32_t W,
                                                              int32_t shared, int32_t vec) {
    const int64_t r = blockIdx.y;
    const int32_t j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (j0 >= width) return;
    const int32_t n = lens[r], end = *indexed_end, take = takes[r];
    const UnionBounds x = union_bounds(n, end, S, W);
    const int32_t hist = take * 64;
    const int32_t sp = (x.s + 63) / 64, tp = max(sp, x.t / 64);
    const float* row = raw + r * raw_stride;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int32_t j = j0 + q;
        bool valid;
        int32_t source = j;
        if (j < hist) {
            const int32_t pi = j / 64;
            const int64_t page = pi < max_take ? selected[r * max_take + pi] : -1;
            const int32_t member = (page >= 0 && page < members_pages) ? members[page * 64 + j % 64] : -1;
            valid = member >= x.s && member < x.t && member < n && member < end;
        } else {
            const int32_t k = j - hist;
            valid = k < x.c;
            if (shared) {
                const int32_t logical = k < x.s ? k : x.t + k - x.s;
                source = hist + (logical < sp * 64 ? logical : sp * 64 + logical - tp * 64);
            }
        }
        v[q] = (valid && j < width && source >= 0 && source < raw_cols) ? row[source] : -__builtin_inff();
    }
    float* dst = out + r * width + j0;
    if (vec) {
        *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (j0 + q < width) dst[q] = v[q];
    }
}

// kernels.py:62-76: Top-K candidate ids -> logical token (history member,
// sink or tail position) -> physical slot nt[logical / 64] * 64 + logical % 64;
// -1 for -inf values and positions outside [0, n).  Without `values`, the
// value of id i is read from the canonical scores (scores[r, i], -inf past
// score_cols), which is what the Top-K selected it from.
__global__ __launch_bounds__(256) void union_map_topk_kernel(const void* __restrict__ ids, int32_t ids64,
                                                             const float* __restrict__ values,
                                                             const float* __restrict__ scores, int64_t score_stride,
                                                             int32_t score_cols,
                                                             const int32_t* __restrict__ lens,
                                                             const int32_t* __restrict__ indexed_end,
                                                             const int32_t* __restrict__ takes,
                                                             const int32_t* __restrict__ selected,
                                                             const int32_t* __restrict__ members,
                                                             int64_t members_pages, const int32_t* __restrict__ nt,
                                                             int32_t nt_len, int32_t* __restrict__ logical_out,
                                                             int32_t* __restrict__ slots, int32_t max_take,
                                                             int32_t top, int32_t S, int32_t W) {
    const int64_t r = blockIdx.y;
    const int32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= top) return;
    const int64_t at = r * top + i;
    const int32_t rank = ids64 ? (int32_t)static_cast<const int64_t*>(ids)[at] : static_cast<const int32_t*>(ids)[at];
    const float value = values ? values[at]
                               : (rank >= 0 && rank < score_cols ? scores[r * score_stride + rank] : -__builtin_inff());
    const int32_t take = takes[r], n = lens[r];
    const UnionBounds x = union_bounds(n, *indexed_end, S, W);
    int32_t logical;
    if (rank < take * 64) {
        int32_t member = -1;
        if (rank >= 0) {
            const int32_t pi = rank / 64;
            const int64_t page = pi < max_take ? selected[r * max_take + pi] : -1;
            if (page >= 0 && page < members_pages) member = members[page * 64 + rank % 64];
        }
        logical = member;
    } else {
        const int32_t k = rank - take * 64;
        logical = k < x.s ? k : x.t + k - x.s;
    }
    const bool valid = value != -__builtin_inff() && logical >= 0 && logical < n && logical / 64 < nt_len;
    logical_out[at] = valid ? logical : -1;
    slots[at] = valid ? nt[logical / 64] * 64 + logical % 64 : -1;
}

// Split scoring of the shared chunk: every row scored once against all history
// pages (hist_scores [rows, >= 64 * hist_pages], position = page * 64 + slot)
// and once against the union in its own coordinates (union_scores
// [rows, >= span], union position = up * 64 + slot with up = lp for sink
// pages, sp + lp - tp for tail pages: union.py:33-35).  union_spans gives each
// row's span there (the end of its last candidate) for the shared-table
// scoring; normalize_split gathers the canonical candidate order from the two.
__global__ __launch_bounds__(256) void union_spans_kernel(const int32_t* __restrict__ lens,
                                                          const int32_t* __restrict__ indexed_end,
                                                          const int32_t* __restrict__ desc, int32_t* __restrict__ spans,
                                                          int32_t rows, int32_t S, int32_t W) {
    const int32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const int32_t n = lens[r];
    const UnionBounds x = union_bounds(n, *indexed_end, S, W);
    const int32_t sp = desc[0], tp = desc[1], total = desc[3];
    const int32_t span = x.t < n ? sp * 64 + n - tp * 64 : x.s;
    spans[r] = max(1, min(max(span, x.s), total * 64));
}

__global__ __launch_bounds__(256) void union_normalize_split_kernel(
    const float* __restrict__ hist, int64_t hist_stride, int32_t hist_cols, const float* __restrict__ uni,
    int64_t uni_stride, int32_t uni_cols, const int32_t* __restrict__ lens, const int32_t* __restrict__ indexed_end,
    const int32_t* __restrict__ takes, const int32_t* __restrict__ selected, const int32_t* __restrict__ members,
    int64_t members_pages, const int32_t* __restrict__ desc, float* __restrict__ out, int32_t max_take, int32_t width,
    int32_t S, int32_t W, int32_t vec) {
    // four consecutive candidates per thread (one 16-byte store when the row allows it)
    const int64_t r = blockIdx.y;
    const int32_t j0 = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (j0 >= width) return;
    const int32_t n = lens[r], end = *indexed_end, take = takes[r];
    const UnionBounds x = union_bounds(n, end, S, W);
    const int32_t hist_n = take * 64, sp = desc[0], tp = desc[1];
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int32_t j = j0 + q;
        v[q] = -__builtin_inff();
        if (j >= width) continue;
        if (j < hist_n) {
            const int32_t pi = j / 64;
            const int64_t page = pi < max_take ? selected[r * max_take + pi] : -1;
            const int32_t member = (page >= 0 && page < members_pages) ? members[page * 64 + j % 64] : -1;
            const int64_t pos = page * 64 + j % 64;
            if (member >= x.s && member < x.t && member < n && member < end && pos < hist_cols)
                v[q] = hist[r * hist_stride + pos];
        } else if (j - hist_n < x.c) {
            const int32_t k = j - hist_n;
            const int32_t logical = k < x.s ? k : x.t + k - x.s;
            const int32_t lp = logical / 64;
            const int64_t pos = (int64_t)(lp < sp ? lp : sp + lp - tp) * 64 + logical % 64;
            if (pos >= 0 && pos < uni_cols) v[q] = uni[r * uni_stride + pos];
        }
    }
    float* dst = out + r * width + j0;
    if (vec) {
        *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (j0 + q < width) dst[q] = v[q];
    }
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_stage_union(const void* src, int64_t src_pages, const int32_t* nt, int32_t nt_len,
                              const int32_t* lens, int32_t rows, const int32_t* indexed_end, void* dst,
                              int32_t dst_pages, int32_t* meta, int32_t* desc, int32_t sink, int32_t window,
                              void* stream) {
    V1_REQUIRE(rows >= 1 && dst_pages >= 0 && nt_len >= 0 && src_pages >= 0 && sink >= 0 && window >= 0,
               "stage_union: bad shape");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0,
               "stage_union: pools must be 16-byte aligned");
    V1_REQUIRE(src && nt && lens && indexed_end && meta && desc && (dst || dst_pages == 0), "stage_union: null buffer");
    hipLaunchKernelGGL(stage_union_kernel, dim3((uint32_t)(dst_pages + cdiv(rows, 256))), dim3(256), 0,
                       as_stream(stream), static_cast<const uint8_t*>(src), src_pages, nt, nt_len, lens, rows,
                       indexed_end, static_cast<uint8_t*>(dst), dst_pages, meta, desc, sink, window);
    return V1_LAUNCHED("stage_union");
}

extern "C" int v1_union_tables(const int32_t* lens, const int32_t* indexed_end, const int32_t* takes,
                               const int32_t* selected, const int32_t* desc, int32_t* ft, int32_t* dg_lens,
                               int32_t* clens, int32_t rows, int32_t cap, int32_t max_take, int32_t scratch,
                               int32_t fp, int32_t sink, int32_t window, int32_t shared, void* stream) {
    V1_REQUIRE(rows >= 0 && max_take >= 0 && fp >= 0 && sink >= 0 && window >= 0, "tables: bad shape");
    V1_REQUIRE(!shared || desc, "tables: shared mode needs the union descriptor");
    if (rows == 0) return V1_OK;
    hipLaunchKernelGGL(union_tables_kernel, dim3((uint32_t)rows), dim3(256), 0, as_stream(stream), lens, indexed_end,
                       takes, selected, desc, ft, dg_lens, clens, cap, max_take, scratch, fp, sink, window, shared);
    return V1_LAUNCHED("tables");
}

extern "C" int v1_union_normalize(const float* raw, int64_t raw_stride, int32_t raw_cols, const int32_t* lens,
                                  const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                                  const int32_t* members, int64_t members_pages, float* out, int32_t rows,
                                  int32_t max_take, int32_t width, int32_t sink, int32_t window, int32_t shared,
                                  void* stream) {
    V1_REQUIRE(rows >= 0 && width >= 0 && raw_cols >= 0 && max_take >= 0, "normalize: bad shape");
    if (rows == 0 || width == 0) return V1_OK;
    const int32_t vec = (width % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) ? 1 : 0;
    hipLaunchKernelGGL(union_normalize_kernel, dim3((uint32_t)cdiv(cdiv(width, 4), 256), (uint32_t)rows), dim3(256),
                       0, as_stream(stream), raw, raw_stride, raw_cols, lens, indexed_end, takes, selected, members,
                       members_pages, out, max_take, width, sink, window, shared, vec);
    return V1_LAUNCHED("normalize");
}

extern "C" int v1_union_map_topk(const void* ids, int32_t ids_bits, const float* values, const float* scores,
                                 int64_t score_stride, int32_t score_cols, const int32_t* lens,
                                 const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                                 const int32_t* members, int64_t members_pages, const int32_t* nt, int32_t nt_len,
                                 int32_t* logical, int32_t* slots, int32_t rows, int32_t max_take, int32_t top,
                                 int32_t sink, int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && top >= 0 && max_take >= 0 && nt_len >= 0, "map_topk: bad shape");
    V1_REQUIRE(ids_bits == 32 || ids_bits == 64, "map_topk: ids must be int32 or int64");
    V1_REQUIRE(values || scores, "map_topk: values or canonical scores are required");
    if (rows == 0 || top == 0) return V1_OK;
    hipLaunchKernelGGL(union_map_topk_kernel, dim3((uint32_t)cdiv(top, 256), (uint32_t)rows), dim3(256), 0,
                       as_stream(stream), ids, ids_bits == 64 ? 1 : 0, values, scores, score_stride, score_cols,
                       lens, indexed_end, takes, selected,
                       members, members_pages, nt, nt_len, logical, slots, max_take, top, sink, window);
    return V1_LAUNCHED("map_topk");
}

extern "C" int v1_union_spans(const int32_t* lens, const int32_t* indexed_end, const int32_t* desc, int32_t* spans,
                              int32_t rows, int32_t sink, int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && sink >= 0 && window >= 0, "union_spans: bad shape");
    if (rows == 0) return V1_OK;
    hipLaunchKernelGGL(union_spans_kernel, dim3((uint32_t)cdiv(rows, 256)), dim3(256), 0, as_stream(stream), lens,
                       indexed_end, desc, spans, rows, sink, window);
    return V1_LAUNCHED("union_spans");
}

extern "C" int v1_union_normalize_split(const float* hist, int64_t hist_stride, int32_t hist_cols, const float* uni,
                                        int64_t uni_stride, int32_t uni_cols, const int32_t* lens,
                                        const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                                        const int32_t* members, int64_t members_pages, const int32_t* desc, float* out,
                                        int32_t rows, int32_t max_take, int32_t width, int32_t sink, int32_t window,
                                        void* stream) {
    V1_REQUIRE(rows >= 0 && width >= 0 && hist_cols >= 0 && uni_cols >= 0 && max_take >= 0,
               "normalize_split: bad shape");
    if (rows == 0 || width == 0) return V1_OK;
    const int32_t vec = (width % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) ? 1 : 0;
    hipLaunchKernelGGL(union_normalize_split_kernel, dim3((uint32_t)cdiv(cdiv(width, 4), 256), (uint32_t)rows),
                       dim3(256), 0, as_stream(stream), hist, hist_stride, hist_cols, uni, uni_stride, uni_cols, lens,
                       indexed_end, takes, selected, members, members_pages, desc, out, max_take, width, sink, window,
                       vec);
    return V1_LAUNCHED("normalize_split");
}
