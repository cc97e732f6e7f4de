// Page manager (fingerprint / match_pages / allocate / publish / release),
// query metadata, fine page tables and shared tail staging.
// Semantics: sglang/srt/layers/attention/v1_deepseek/kernels.py:57-179 (page
// manager), :224-245, :379-441, :488-591 (metadata, tables, staging).
// All integer work; the byte movers use 16-byte vector accesses.
#include "common.h"

namespace v1 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Block (256 threads) sum of two int64 values; result valid in thread 0.
__device__ __forceinline__ void block_sum2(int64_t& a, int64_t& b) {
    __shared__ int64_t sa[4], sb[4];
    a = wave_sum64(a);
    b = wave_sum64(b);
    const int w = threadIdx.x / kWave;
    if (__lane_id() == 0) {
        sa[w] = a;
        sb[w] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a = sa[0] + sa[1] + sa[2] + sa[3];
        b = sb[0] + sb[1] + sb[2] + sb[3];
    }
}

// h0 = sum x_i (i+1) + sum m * 104729 ;  h1 = sum x_i (i+7) 1000003 + sum m_i (i+1) 65537
// over the page bytes x and its 64 members m (kernels.py:57-69).  Integer sums:
// the order of accumulation does not change the result.
__global__ __launch_bounds__(256) void fingerprint_kernel(const uint8_t* tmp, const int32_t* map, const int32_t* meta,
                                                          int64_t* hash, int64_t page_bytes) {
    if (meta[2] == 0) return;
    const int64_t p = blockIdx.x;
    const uint8_t* x = tmp + p * page_bytes;
    int64_t xw = 0, xs = 0;  // sum x_i (i+1), sum x_i
    for (int64_t i = threadIdx.x; i < page_bytes; i += 256) {
        const int64_t v = x[i];
        xw += v * (i + 1);
        xs += v;
    }
    int64_t ms = 0, mw = 0;
    if (threadIdx.x < 64) {
        const int64_t m = map[p * 64 + threadIdx.x];
        ms = m;
        mw = m * (threadIdx.x + 1);
    }
    int64_t a = xw, b = xs;
    block_sum2(a, b);
    __syncthreads();
    int64_t c = ms, d = mw;
    block_sum2(c, d);
    if (threadIdx.x == 0) {
        hash[p * 2] = a + c * 104729;
        hash[p * 2 + 1] = (a + 6 * b) * 1000003 + d * 65537;
    }
}

// Lowest live page j > after with equal fingerprints, or capacity.
__device__ int32_t next_candidate(const int32_t* refs, const int64_t* hashes, int64_t h0, int64_t h1,
                                  int32_t capacity, int32_t after) {
    __shared__ int32_t best[4];
    int32_t mine = capacity;
    for (int32_t j = after + 1 + threadIdx.x; j < capacity; j += 256) {
        if (refs[j] > 0 && hashes[2 * (int64_t)j] == h0 && hashes[2 * (int64_t)j + 1] == h1) {
            mine = j;
            break;  // strided scan: first hit of this thread is its minimum
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mine = min(mine, __shfl_xor(mine, off, kWave));
    if (__lane_id() == 0) best[threadIdx.x / kWave] = mine;
    __syncthreads();
    const int32_t r = min(min(best[0], best[1]), min(best[2], best[3]));
    __syncthreads();
    return r;
}

__device__ bool same_page(const uint8_t* a, const uint8_t* b, int64_t page_bytes, const int32_t* ma,
                          const int32_t* mb) {
    __shared__ int diff;
    if (threadIdx.x == 0) diff = 0;
    __syncthreads();
    bool d = false;
    if ((page_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0) {
        const u32x4* va = reinterpret_cast<const u32x4*>(a);
        const u32x4* vb = reinterpret_cast<const u32x4*>(b);
        for (int64_t i = threadIdx.x; i < page_bytes / 16; i += 256) {
            const u32x4 x = va[i], y = vb[i];
            d |= x.x != y.x || x.y != y.y || x.z != y.z || x.w != y.w;
        }
    } else {
        for (int64_t i = threadIdx.x; i < page_bytes; i += 256) d |= a[i] != b[i];
    }
    if (threadIdx.x < 64) d |= ma[threadIdx.x] != mb[threadIdx.x];
    if (d) diff = 1;
    __syncthreads();
    const bool same = diff == 0;
    __syncthreads();
    return same;
}

// kernels.py:72-113: lowest live page with equal fingerprints AND equal bytes
// and members; otherwise -1.
__global__ __launch_bounds__(256) void match_kernel(const uint8_t* tmp, const int32_t* map, const int64_t* hash,
                                                    const int32_t* meta, const uint8_t* fine, const int32_t* members,
                                                    const int64_t* hashes, const int32_t* refs, int32_t* match,
                                                    int32_t capacity, int64_t page_bytes) {
    if (meta[2] == 0) return;
    const int64_t p = blockIdx.x;
    const int64_t h0 = hash[2 * p], h1 = hash[2 * p + 1];
    int32_t found = -1;
    int32_t cand = next_candidate(refs, hashes, h0, h1, capacity, -1);
    while (cand < capacity) {
        if (same_page(tmp + p * page_bytes, fine + (int64_t)cand * page_bytes, page_bytes, map + p * 64,
                      members + (int64_t)cand * 64)) {
            found = cand;
            break;
        }
        cand = next_candidate(refs, hashes, h0, h1, capacity, cand);
    }
    if (threadIdx.x == 0) match[p] = found;
}

// kernels.py:116-131 for one record of `pages` pages (one wave, pages <= 64).
__global__ void allocate_kernel(const int32_t* meta, const int32_t* match, int32_t* free_stack, int32_t* count,
                                int32_t* refs, int32_t* tables, uint8_t* fresh, int32_t pages, int32_t* status) {
    if (meta[2] == 0) return;
    const int i = threadIdx.x;
    const bool in = i < pages;
    const int32_t m = in ? match[i] : 0;
    const bool f = in && m < 0;
    const uint64_t ballot = __ballot(f);
    const int32_t rank = (int32_t)lanes_below(ballot);
    const int32_t needed = (int32_t)popc64(ballot);
    const int32_t c = *count;
    if (c < needed) {  // arena exhausted: the reference asserts; report and leave state untouched
        if (i == 0 && status != nullptr) atomicOr(status, 1);
        return;
    }
    if (in) {
        const int32_t dst = f ? free_stack[c - 1 - rank] : m;
        atomicAdd(&refs[dst], 1);
        tables[(int64_t)meta[1] * pages + i] = dst;
        fresh[i] = f ? 1 : 0;
    }
    __syncthreads();
    if (i == 0) *count = c - needed;
}

// kernels.py:134-167: copy new pages (bytes, members, fingerprints) to their
// slot; always copy the record's 8 centers of page p (128 FP8 bytes + scale).
__global__ __launch_bounds__(256) void publish_kernel(const uint8_t* tmp, const uint8_t* tc, const int32_t* map,
                                                      const int64_t* hash, const int32_t* meta, const int32_t* tables,
                                                      const uint8_t* fresh, uint8_t* fine, uint8_t* centers,
                                                      int32_t* members, int64_t* hashes, int32_t pages,
                                                      int64_t page_bytes) {
    if (meta[2] == 0) return;
    const int64_t p = blockIdx.x;
    const int64_t lease = meta[1];
    if (fresh[p]) {
        const int64_t dst = tables[lease * pages + p];
        const uint8_t* s = tmp + p * page_bytes;
        uint8_t* d = fine + dst * page_bytes;
        if ((page_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(d)) & 15) == 0) {
            for (int64_t i = threadIdx.x; i < page_bytes / 16; i += 256)
                reinterpret_cast<u32x4*>(d)[i] = reinterpret_cast<const u32x4*>(s)[i];
        } else {
            for (int64_t i = threadIdx.x; i < page_bytes; i += 256) d[i] = s[i];
        }
        if (threadIdx.x < 64) members[dst * 64 + threadIdx.x] = map[p * 64 + threadIdx.x];
        if (threadIdx.x < 2) hashes[dst * 2 + threadIdx.x] = hash[p * 2 + threadIdx.x];
    }
    if (tc != nullptr) {
        // 8 centers x 128 bytes, then their 8 scales
        for (int x = threadIdx.x; x < 8 * 128; x += 256) {
            const int64_t sc = p * 8 + x / 128;
            const int64_t dc = lease * pages * 8 + sc;
            centers[(dc / 64) * 8448 + (dc % 64) * 128 + (x % 128)] = tc[(sc / 64) * 8448 + (sc % 64) * 128 + (x % 128)];
        }
        if (threadIdx.x < 8) {
            const int64_t sc = p * 8 + threadIdx.x;
            const int64_t dc = lease * pages * 8 + sc;
            reinterpret_cast<float*>(centers)[(dc / 64) * 2112 + 2048 + dc % 64] =
                reinterpret_cast<const float*>(tc)[(sc / 64) * 2112 + 2048 + sc % 64];
        }
    }
}

// kernels.py:170-179; duplicate pages in one table are decremented in table
// order (the last decrement of a page frees it), so the pushed order is fixed.
__global__ void release_kernel(const int32_t* table, int32_t* refs, int32_t* free_stack, int32_t* count,
                               int32_t pages) {
    __shared__ int32_t dead[64];
    if (threadIdx.x != 0) return;
    int32_t n = 0;
    for (int i = 0; i < pages; ++i) {
        const int32_t page = table[i];
        const int32_t old = atomicAdd(&refs[page], -1);
        if (old == 1) dead[n++] = page;
    }
    const int32_t base = atomicAdd(count, n);
    for (int i = 0; i < n; ++i) free_stack[base + i] = dead[i];
}

struct Geometry {
    int32_t n, pages, take, sink, tail, fine;
};

__device__ __forceinline__ Geometry geometry(int32_t n, int32_t topk, int32_t num, int32_t den, int32_t sink_cap,
                                             int32_t window) {
    Geometry g;
    g.n = n;
    g.pages = max(n - 1, 0) / 1024 * 16;
    const int64_t frac = ((int64_t)g.pages * num + den - 1) / den;
    const int64_t floor_take = (topk + 63) / 64;
    g.take = (int32_t)min((int64_t)g.pages, max(frac, floor_take));
    g.sink = min(sink_cap, n);
    g.tail = max(g.sink, min(max(n - 1, 0) / 1024 * 1024, max(g.sink, n - window)));
    g.fine = g.take * 64 + g.sink + n - g.tail;
    return g;
}

// kernels.py:568-591 (one wave per row: 128 tail-page checks, 2 per lane)
__global__ void query_metadata_kernel(const int32_t* lens, const int32_t* nt, int32_t* fine_lens, int32_t* takes,
                                      int32_t* dg_lens, int32_t* center_lens, int32_t* tail_rows, int32_t np,
                                      int32_t topk, int32_t num, int32_t den, int32_t sink_cap, int32_t window) {
    const int64_t row = blockIdx.x;
    const int32_t n = lens[row];
    const Geometry g = geometry(n, topk, num, den, sink_cap, window);
    const int lane = threadIdx.x;
    if (lane == 0) {
        fine_lens[row] = g.fine;
        takes[row] = g.take;
        dg_lens[row] = max(g.fine, 1);
        center_lens[row] = max(g.pages * 8, 1);
    }
    bool differ = false;
    for (int i = lane; i < 128; i += kWave) {
        const int32_t page = i == 0 ? 0 : g.tail / 64 + i - 1;
        const bool valid = n > 0 && (i == 0 || page < (n + 63) / 64) && page < np;
        const int32_t mine = valid ? nt[row * np + page] : -1;
        const int32_t first = valid ? nt[page] : -1;
        differ |= mine != first;
    }
    const bool share = n == lens[0] && __ballot(differ) == 0;
    if (lane == 0) tail_rows[row] = share ? 0 : (int32_t)row;
}

__global__ void query_lengths_kernel(const int32_t* lens, int32_t* fine_lens, int32_t* takes, int32_t rows,
                                     int32_t topk, int32_t num, int32_t den, int32_t sink_cap, int32_t window) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const Geometry g = geometry(lens[row], topk, num, den, sink_cap, window);
    fine_lens[row] = g.fine;
    takes[row] = g.take;
}

// kernels.py:379-404 (tail_rows == NULL) and :488-514.
__global__ void fine_table_kernel(const int32_t* rt, const void* selected, int32_t sel64, const int32_t* takes,
                                  int32_t* ft, const int32_t* tail_rows, int32_t capacity, int32_t maxp,
                                  int32_t take_stride, int32_t fp, int32_t scratch) {
    const int64_t row = blockIdx.x;
    const int32_t take = takes[row];
    const int64_t owner = tail_rows ? tail_rows[row] : row;
    for (int32_t j = threadIdx.x; j < fp; j += blockDim.x) {
        int32_t page;
        if (j < take) {
            int32_t rank = 0;
            if (j < take_stride)
                rank = sel64 ? (int32_t) static_cast<const int64_t*>(selected)[row * take_stride + j]
                             : static_cast<const int32_t*>(selected)[row * take_stride + j];
            page = (rank >= 0 && rank < maxp) ? rt[row * maxp + rank] : 0;
        } else {
            page = (int32_t)(capacity + owner * scratch + min(max(j - take, 0), scratch - 1));
        }
        ft[row * fp + j] = page;
    }
}

// kernels.py:518-564 (tail_rows == NULL: every row owns its scratch, :407-441).
// Block (row, g): copies tail-candidate pages kPages*g .. +kPages-1 of an
// owner row, 64 tokens x (128 FP8 bytes + fp32 scale) each; slots past the
// candidate count become zero, pages past it (other than page 0) are left
// untouched.  Every thread issues its page-table reads, then its 2*kPages
// 16-byte loads and its scale load, then the stores.  With indexed_end, the
// tail starts at the published index end instead of the last whole
// 1024-token bucket (experiments/tail_union_lab_20261021/
// baseline_published.py:21-61).
// Measured: four pages per work-group for prefill-sized batches (1024 rows of
// 2 or 34 candidate pages: 18.9 -> 8.4 and 18.7 -> 13.3 us, most of the
// one-page grid's work-groups having nothing to copy), one page for a decode
// batch (128 rows of up to 34 pages: 19.2 us, 20.9 with four).
template <int kPages>
__global__ __launch_bounds__(256) void stage_tail_kernel(const uint8_t* native, const int32_t* nt, const int32_t* lens,
                                                         const int32_t* indexed_end, uint8_t* fine,
                                                         const int32_t* tail_rows, int32_t capacity, int32_t np,
                                                         int32_t scratch, int32_t sink_cap, int32_t window,
                                                         int64_t native_pages, int64_t fine_pages) {
    const int64_t row = blockIdx.x;
    constexpr int kChunks = kPages * 64 * 8 / 256;  // 16-byte chunks per thread
    static_assert(kPages >= 1 && kPages <= 4, "one scale slot per thread of the first 64 * kPages");
    const int32_t p0 = blockIdx.y * kPages;
    if (tail_rows != nullptr && tail_rows[row] != row) return;
    const int32_t n = lens[row];
    const int32_t sink = min(n, sink_cap);
    const int32_t indexed = indexed_end ? min(max(*indexed_end, 0), n) : max(n - 1, 0) / 1024 * 1024;
    const int32_t tail = max(sink, min(indexed, max(sink, n - window)));
    const int32_t count = sink + n - tail;
    if (!(p0 * 64 < count || p0 == 0)) return;
    // page p of the row's scratch is written: inside the scratch and the pool,
    // and holding candidates (page 0 always)
    const int64_t dst0 = capacity + row * scratch + p0;
    auto written = [&](int j) {
        const int32_t p = p0 + j;
        return p < scratch && (p * 64 < count || p == 0) && dst0 + j < fine_pages;
    };
    // the 128 key bytes of candidate slot i in the native pool (nullptr: a
    // zero slot: past the count, or its page outside the table or the pool)
    auto key_row = [&](int32_t i) -> const uint8_t* {
        if (i >= count) return nullptr;
        const int32_t logical = i < sink ? i : tail + i - sink;
        const int32_t e = logical / 64;
        const int64_t page = e < np ? nt[row * np + e] : -1;
        if (page < 0 || page >= native_pages) return nullptr;
        return native + page * V1_PAGE_BYTES + (logical % 64) * 128;
    };
    // chunk k of this thread: page p0 + c / 512, slot (c % 512) / 8, part c % 8
    // with c = threadIdx.x + 256 k; the thread's scale is slot threadIdx.x % 64
    // of page p0 + threadIdx.x / 64
    const int t = (int)threadIdx.x;
    const uint8_t* src[kChunks];
#pragma unroll
    for (int k = 0; k < kChunks; ++k) src[k] = key_row((p0 + k / 2) * 64 + (t + 256 * (k % 2)) / 8);
    const bool has_scale = t < 64 * kPages;
    const uint8_t* ssrc = has_scale ? key_row((p0 + t / 64) * 64 + t % 64) : nullptr;
    u32x4 v[kChunks];
#pragma unroll
    for (int k = 0; k < kChunks; ++k)
        v[k] = src[k] ? reinterpret_cast<const u32x4*>(src[k])[t % 8] : u32x4{0u, 0u, 0u, 0u};
    // (the scale of the key row at token j of a page lies at byte 8192 + 4 j)
    const int32_t si = (p0 + t / 64) * 64 + t % 64;
    const int32_t sj = (si < sink ? si : tail + si - sink) % 64;
    const float sc = ssrc ? reinterpret_cast<const float*>(ssrc - sj * 128 + 8192)[sj] : 0.f;
#pragma unroll
    for (int k = 0; k < kChunks; ++k)
        if (written(k / 2))
            reinterpret_cast<u32x4*>(fine + (dst0 + k / 2) * V1_PAGE_BYTES + ((t + 256 * (k % 2)) / 8) * 128)[t % 8] = v[k];
    if (has_scale && written(t / 64)) reinterpret_cast<float*>(fine + (dst0 + t / 64) * V1_PAGE_BYTES + 8192)[t % 64] = sc;
}

// stage_tail over pages of 64 rows of row_bytes each (MLA latent rows of 656
// bytes: 512 FP8 + 64 bf16 RoPE + fp32 scales), the same slot rule as
// stage_tail_kernel with one contiguous row per token instead of 128 key bytes
// plus a separate scale.  Rows are 16-byte multiples; chunk c of the page is
// part c % parts of slot c / parts.
__global__ __launch_bounds__(256) void stage_tail_rows_kernel(const uint8_t* native, const int32_t* nt,
                                                              const int32_t* lens, uint8_t* fine,
                                                              const int32_t* tail_rows, int32_t capacity, int32_t np,
                                                              int32_t scratch, int32_t sink_cap, int32_t window,
                                                              int64_t native_pages, int64_t fine_pages,
                                                              int32_t row_bytes) {
    const int64_t row = blockIdx.x;
    const int32_t p = blockIdx.y;
    if (tail_rows != nullptr && tail_rows[row] != row) return;
    const int32_t n = lens[row];
    const int32_t sink = min(n, sink_cap);
    const int32_t tail = max(sink, min(max(n - 1, 0) / 1024 * 1024, max(sink, n - window)));
    const int32_t count = sink + n - tail;
    if (!(p * 64 < count || p == 0)) return;
    const int64_t dst = capacity + row * scratch + p;
    if (dst >= fine_pages) return;
    const int64_t page_bytes = (int64_t)row_bytes * 64;
    const int32_t parts = row_bytes / 16;
    const int32_t total = 64 * parts;
    u32x4* out = reinterpret_cast<u32x4*>(fine + dst * page_bytes);
    // kBatch chunks per thread at a time: their sources first (page-table
    // reads), then all their loads, then the stores
    constexpr int kBatch = 8;
    for (int32_t c0 = threadIdx.x; c0 < total; c0 += 256 * kBatch) {
        const u32x4* src[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int32_t c = c0 + 256 * k;
            const int32_t slot = c / parts, part = c - slot * parts;
            const int32_t i = p * 64 + slot;
            src[k] = nullptr;
            if (c < total && i < count) {
                const int32_t logical = i < sink ? i : tail + i - sink;
                const int32_t e = logical / 64;
                const int64_t page = e < np ? nt[row * np + e] : -1;
                if (page >= 0 && page < native_pages)
                    src[k] = reinterpret_cast<const u32x4*>(native + page * page_bytes +
                                                            (int64_t)(logical % 64) * row_bytes) + part;
            }
        }
        u32x4 v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = src[k] ? *src[k] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            if (c0 + 256 * k < total) out[c0 + 256 * k] = v[k];
    }
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_fingerprint(const uint8_t* tmp, const int32_t* map, const int32_t* meta, int64_t* hash,
                              int32_t pages, int64_t page_bytes, void* stream) {
    V1_REQUIRE(pages >= 0 && page_bytes > 0, "fingerprint: bad shape");
    if (pages == 0) return V1_OK;
    hipLaunchKernelGGL(fingerprint_kernel, dim3(pages), dim3(256), 0, as_stream(stream), tmp, map, meta, hash,
                       page_bytes);
    return V1_LAUNCHED("fingerprint");
}

extern "C" int v1_match_pages(const uint8_t* tmp, const int32_t* map, const int64_t* hash, const int32_t* meta,
                              const uint8_t* fine, const int32_t* members, const int64_t* hashes, const int32_t* refs,
                              int32_t* match, int32_t pages, int32_t capacity, int64_t page_bytes, void* stream) {
    V1_REQUIRE(pages >= 0 && capacity > 0 && page_bytes > 0, "match_pages: bad shape");
    if (pages == 0) return V1_OK;
    hipLaunchKernelGGL(match_kernel, dim3(pages), dim3(256), 0, as_stream(stream), tmp, map, hash, meta, fine,
                       members, hashes, refs, match, capacity, page_bytes);
    return V1_LAUNCHED("match_pages");
}

extern "C" int v1_allocate(const int32_t* meta, const int32_t* match, int32_t* free_stack, int32_t* count,
                           int32_t* refs, int32_t* tables, uint8_t* fresh, int32_t pages, int32_t* status,
                           void* stream) {
    V1_REQUIRE(pages > 0 && pages <= 64, "allocate: pages must be in [1, 64]");
    hipLaunchKernelGGL(allocate_kernel, dim3(1), dim3(kWave), 0, as_stream(stream), meta, match, free_stack, count,
                       refs, tables, fresh, pages, status);
    return V1_LAUNCHED("allocate");
}

extern "C" int v1_publish(const uint8_t* tmp, const uint8_t* centers_src, const int32_t* map, const int64_t* hash,
                          const int32_t* meta, const int32_t* tables, const uint8_t* fresh, uint8_t* fine,
                          uint8_t* centers, int32_t* members, int64_t* hashes, int32_t pages, int64_t page_bytes,
                          void* stream) {
    V1_REQUIRE(pages >= 0 && page_bytes > 0, "publish: bad shape");
    V1_REQUIRE(centers_src == nullptr || centers != nullptr, "publish: centers destination missing");
    if (pages == 0) return V1_OK;
    hipLaunchKernelGGL(publish_kernel, dim3(pages), dim3(256), 0, as_stream(stream), tmp, centers_src, map, hash,
                       meta, tables, fresh, fine, centers, members, hashes, pages, page_bytes);
    return V1_LAUNCHED("publish");
}

extern "C" int v1_release(const int32_t* table, int32_t* refs, int32_t* free_stack, int32_t* count, int32_t pages,
                          void* stream) {
    V1_REQUIRE(pages > 0 && pages <= 64, "release: pages must be in [1, 64]");
    hipLaunchKernelGGL(release_kernel, dim3(1), dim3(kWave), 0, as_stream(stream), table, refs, free_stack, count,
                       pages);
    return V1_LAUNCHED("release");
}

extern "C" int v1_query_metadata(const int32_t* lens, const int32_t* nt, int32_t* fine_lens, int32_t* takes,
                                 int32_t* dg_lens, int32_t* center_lens, int32_t* tail_rows, int32_t rows, int32_t np,
                                 int32_t topk, int32_t num, int32_t den, int32_t sink, int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && np > 0 && den > 0, "query_metadata: bad shape");
    if (rows == 0) return V1_OK;
    hipLaunchKernelGGL(query_metadata_kernel, dim3(rows), dim3(kWave), 0, as_stream(stream), lens, nt, fine_lens, takes,
                       dg_lens, center_lens, tail_rows, np, topk, num, den, sink, window);
    return V1_LAUNCHED("query_metadata");
}

extern "C" int v1_query_lengths(const int32_t* lens, int32_t* fine_lens, int32_t* takes, int32_t rows, int32_t topk,
                                int32_t num, int32_t den, int32_t sink, int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && den > 0, "query_lengths: bad shape");
    if (rows == 0) return V1_OK;
    hipLaunchKernelGGL(query_lengths_kernel, dim3((uint32_t)cdiv(rows, 256)), dim3(256), 0, as_stream(stream), lens,
                       fine_lens, takes, rows, topk, num, den, sink, window);
    return V1_LAUNCHED("query_lengths");
}

extern "C" int v1_fine_table(const int32_t* rt, const void* selected, int32_t selected_bits, const int32_t* takes,
                             int32_t* ft, const int32_t* tail_rows, int32_t rows, int32_t capacity, int32_t maxp,
                             int32_t take_stride, int32_t fp, int32_t scratch, void* stream) {
    V1_REQUIRE(rows >= 0 && fp >= 0 && maxp > 0 && scratch > 0, "fine_table: bad shape");
    V1_REQUIRE(selected_bits == 32 || selected_bits == 64, "fine_table: selected must be int32 or int64");
    if (rows == 0 || fp == 0) return V1_OK;
    hipLaunchKernelGGL(fine_table_kernel, dim3(rows), dim3(256), 0, as_stream(stream), rt, selected,
                       selected_bits == 64, takes, ft, tail_rows, capacity, maxp, take_stride, fp, scratch);
    return V1_LAUNCHED("fine_table");
}

// Four pages per work-group from 512 rows on (prefill-sized batches), one
// below (decode batches: more, shorter work-groups keep more of the rows'
// pages in flight at once).
static void launch_stage_tail(const uint8_t* native, const int32_t* nt, const int32_t* lens,
                              const int32_t* indexed_end, uint8_t* fine, const int32_t* tail_rows, int32_t rows,
                              int32_t capacity, int32_t np, int32_t scratch, int32_t sink, int32_t window,
                              int64_t native_pages, int64_t fine_pages, hipStream_t st) {
    if (rows >= 512)
        hipLaunchKernelGGL(stage_tail_kernel<4>, dim3(rows, (uint32_t)cdiv(scratch, 4)), dim3(256), 0, st, native, nt,
                           lens, indexed_end, fine, tail_rows, capacity, np, scratch, sink, window, native_pages,
                           fine_pages);
    else
        hipLaunchKernelGGL(stage_tail_kernel<1>, dim3(rows, scratch), dim3(256), 0, st, native, nt, lens, indexed_end,
                           fine, tail_rows, capacity, np, scratch, sink, window, native_pages, fine_pages);
}

extern "C" int v1_stage_tail(const uint8_t* native, const int32_t* nt, const int32_t* lens, uint8_t* fine,
                             const int32_t* tail_rows, int32_t rows, int32_t capacity, int32_t np, int32_t scratch,
                             int32_t sink, int32_t window, int64_t native_pages, int64_t fine_pages, void* stream) {
    V1_REQUIRE(rows >= 0 && np > 0 && scratch > 0 && capacity >= 0, "stage_tail: bad shape");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(native) & 15) == 0 && (reinterpret_cast<uintptr_t>(fine) & 15) == 0,
               "stage_tail: pools must be 16-byte aligned");
    if (rows == 0) return V1_OK;
    launch_stage_tail(native, nt, lens, nullptr, fine, tail_rows, rows, capacity, np, scratch, sink, window,
                      native_pages, fine_pages, as_stream(stream));
    return V1_LAUNCHED("stage_tail");
}

extern "C" int v1_stage_tail_published(const uint8_t* native, const int32_t* nt, const int32_t* lens,
                                       const int32_t* indexed_end, uint8_t* fine, const int32_t* tail_rows,
                                       int32_t rows, int32_t capacity, int32_t np, int32_t scratch, int32_t sink,
                                       int32_t window, int64_t native_pages, int64_t fine_pages, void* stream) {
    V1_REQUIRE(rows >= 0 && np > 0 && scratch > 0 && capacity >= 0, "stage_tail_published: bad shape");
    V1_REQUIRE(indexed_end != nullptr, "stage_tail_published: indexed_end is required");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(native) & 15) == 0 && (reinterpret_cast<uintptr_t>(fine) & 15) == 0,
               "stage_tail_published: pools must be 16-byte aligned");
    if (rows == 0) return V1_OK;
    launch_stage_tail(native, nt, lens, indexed_end, fine, tail_rows, rows, capacity, np, scratch, sink, window,
                      native_pages, fine_pages, as_stream(stream));
    return V1_LAUNCHED("stage_tail_published");
}

extern "C" int v1_stage_tail_rows(const uint8_t* native, const int32_t* nt, const int32_t* lens, uint8_t* fine,
                                  const int32_t* tail_rows, int32_t rows, int32_t capacity, int32_t np,
                                  int32_t scratch, int32_t sink, int32_t window, int64_t native_pages,
                                  int64_t fine_pages, int32_t row_bytes, void* stream) {
    V1_REQUIRE(rows >= 0 && np > 0 && scratch > 0 && capacity >= 0, "stage_tail_rows: bad shape");
    V1_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "stage_tail_rows: row_bytes must be a positive multiple of 16");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(native) & 15) == 0 && (reinterpret_cast<uintptr_t>(fine) & 15) == 0,
               "stage_tail_rows: pools must be 16-byte aligned");
    if (rows == 0) return V1_OK;
    V1_REQUIRE(native && nt && lens && fine, "stage_tail_rows: null buffer");
    hipLaunchKernelGGL(stage_tail_rows_kernel, dim3(rows, scratch), dim3(256), 0, as_stream(stream), native, nt, lens,
                       fine, tail_rows, capacity, np, scratch, sink, window, native_pages, fine_pages, row_bytes);
    return V1_LAUNCHED("stage_tail_rows");
}
