// Slot gather: copies one source row per (query row, top slot) into a dense
// workspace, zero-filling padding ids.  Pure HBM work: each block first maps
// its tile of slots to source byte offsets in LDS (one id / map lookup per
// slot), then all 256 threads stream the tile as 16-byte chunks so that both
// the workspace writes and the per-row reads are fully coalesced.  Workspace
// stores are non-temporal: the workspace is written once per call and read by
// the attention consumer, while the (smaller) source pool stays cache resident.
//
// Semantics follow sglang/srt/layers/attention/v1_native/kernels.py:62-77.
#include "common.h"

namespace v1 {
namespace {

constexpr int kThreads = 256;
// Tiles, measured on MI355X with 656-byte rows.  When the pool's rows come
// from HBM (a pool well above the caches), 64-slot tiles (42 KB of output)
// beat 256-slot ones by 5%, and copied by 512 threads with 5 loads in flight
// each (one pass over a tile's 2624 chunks) they take 417 us for 1024 x 2048
// rows from a 688 MB pool, against 431 us with 256 threads and 8 loads each
// (32-slot and 128-slot tiles, 1024 threads and 4-8 loads: 418-442 us).  When a small pool stays
// cache-resident, the workspace writes set the pace, and they run fastest with
// few concurrent write streams: 512-slot tiles (336 KB) copied by 1024-thread
// work-groups, one per CU (1.006-1.010 ms for 4096 x 2048 rows against
// 1.034-1.046 ms for 256-slot tiles of 256 threads, eight per CU; two of the
// 1024-thread work-groups per CU take 1.030 ms).  The one-per-CU residency
// is set by reserving more than half of the CU's 160 KB of LDS.
constexpr int kTileSmall = 64;
constexpr int kThreadsSmall = 512;
constexpr int kUnrollSmall = 5;
constexpr int kTileCached = 512;
constexpr int kThreadsCached = 1024;
constexpr size_t kOneWgPerCuLds = 84u << 10;
constexpr int64_t kCachedPoolBytes = 64ll << 20;
constexpr int kUnrollCached = 8;  // independent 16-byte copies in flight per thread

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Source offset of one slot, or -1 for a zero row.
struct RowMap {
    const int32_t* ids;
    int64_t ids_stride;
    int32_t top;
    const int32_t* map;  // NULL: ids are physical rows
    int64_t map_len;
    int64_t map_stride;
    int32_t map_shift;
    int64_t pool_rows;
    int64_t pool_stride_bytes;
    int64_t base_offset_bytes;  // added to every valid row (head offset)

    __device__ __forceinline__ int64_t operator()(int64_t t) const {
        const int64_t r = t / top;
        const int64_t i = t - r * top;
        const int32_t id = ids[r * ids_stride + i];
        if (id < 0) return -1;
        int64_t phys = id;
        if (map != nullptr) {
            const int64_t e = (int64_t)id >> map_shift;
            if (e >= map_len) return -1;
            const int32_t m = map[r * map_stride + e];
            if (m < 0) return -1;
            phys = ((int64_t)m << map_shift) | (id & ((1 << map_shift) - 1));
        }
        if (phys >= pool_rows) return -1;
        return base_offset_bytes + phys * pool_stride_bytes;
    }
};

// Copies `chunks` 16-byte chunks per slot for slots [tile*kTileSlots, ...).
template <int kTileSlots, int kThr, int kUnroll>
__global__ __launch_bounds__(kThr) void gather_rows16(
    const uint8_t* __restrict__ pool, RowMap rm, int64_t total_slots, int32_t chunks,
    uint32_t chunk_magic, int64_t out_row_bytes, uint8_t* __restrict__ out) {
    __shared__ int64_t src[kTileSlots];
    const int64_t first = (int64_t)blockIdx.x * kTileSlots;
    const int tid = threadIdx.x;
    for (int s = tid; s < kTileSlots; s += kThr) {
        const int64_t t = first + s;
        src[s] = t < total_slots ? rm(t) : -1;
    }
    __syncthreads();
    const int64_t left = total_slots - first;
    const int slots = left < kTileSlots ? (int)left : kTileSlots;
    const uint32_t n = (uint32_t)slots * (uint32_t)chunks;
    uint8_t* out_tile = out + first * out_row_bytes;
    for (uint32_t base = 0; base < n; base += kThr * kUnroll) {
        u32x4 v[kUnroll];
        uint32_t g[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            g[u] = base + u * kThr + tid;
            v[u] = u32x4{0u, 0u, 0u, 0u};
            if (g[u] < n) {
                const uint32_t s = chunks == 1 ? g[u] : small_div(g[u], chunk_magic);
                const uint32_t c = g[u] - s * (uint32_t)chunks;
                const int64_t off = src[s];
                if (off >= 0)
                    v[u] = *reinterpret_cast<const u32x4*>(pool + off + (int64_t)c * 16);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (g[u] < n) {
                const uint32_t s = chunks == 1 ? g[u] : small_div(g[u], chunk_magic);
                const uint32_t c = g[u] - s * (uint32_t)chunks;
                u32x4* dst = reinterpret_cast<u32x4*>(out_tile + (int64_t)s * out_row_bytes + (int64_t)c * 16);
                __builtin_nontemporal_store(v[u], dst);
            }
        }
    }
}

// Element-wise fallback for strided rows (any element stride, 128 elements).
template <typename T>
__global__ __launch_bounds__(kThreads) void gather_strided(
    const T* __restrict__ pool, RowMap rm, int64_t total_slots, int64_t elem_stride,
    int32_t dim, T* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t t = idx / dim;
    const int d = (int)(idx - t * dim);
    if (t >= total_slots) return;
    const int64_t off = rm(t);  // element offset (pool_stride_bytes holds elements here)
    out[t * dim + d] = off >= 0 ? pool[off + d * elem_stride] : T(0);
}

int launch_rows(const uint8_t* pool, const RowMap& rm, int64_t total, int64_t row_bytes, int64_t pool_bytes,
                uint8_t* out, hipStream_t st) {
    if (total == 0) return V1_OK;
    const int32_t chunks = (int32_t)(row_bytes / 16);
    const uint32_t magic = chunks == 1 ? 0u : small_div_magic((uint32_t)chunks);
    if (pool_bytes > kCachedPoolBytes)
        hipLaunchKernelGGL((gather_rows16<kTileSmall, kThreadsSmall, kUnrollSmall>), dim3((uint32_t)cdiv(total, kTileSmall)),
                           dim3(kThreadsSmall), 0, st, pool, rm, total, chunks, magic, row_bytes, out);
    else
        hipLaunchKernelGGL((gather_rows16<kTileCached, kThreadsCached, kUnrollCached>), dim3((uint32_t)cdiv(total, kTileCached)),
                           dim3(kThreadsCached), kOneWgPerCuLds, st, pool, rm, total, chunks, magic, row_bytes, out);
    return V1_LAUNCHED("gather_rows16");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_gather_rows(const void* pool, int64_t pool_rows, int64_t row_bytes,
                              int64_t pool_stride_bytes, const int32_t* map, int64_t map_len,
                              int64_t map_stride, int32_t map_shift, const int32_t* ids,
                              int64_t ids_stride, int32_t rows, int32_t top, void* out,
                              void* stream) {
    V1_REQUIRE(rows >= 0 && top >= 0, "gather_rows: negative shape");
    V1_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0 && row_bytes / 16 < 4096,
               "gather_rows: row_bytes must be a positive multiple of 16 (got %lld)", (long long)row_bytes);
    V1_REQUIRE(pool_stride_bytes % 16 == 0 && pool_stride_bytes >= row_bytes,
               "gather_rows: pool stride must be a multiple of 16 and >= row_bytes");
    V1_REQUIRE(aligned16(pool) && aligned16(out), "gather_rows: pool and out must be 16-byte aligned");
    V1_REQUIRE(map_shift >= 0 && map_shift < 31, "gather_rows: bad map_shift");
    V1_REQUIRE(map == nullptr || map_len > 0, "gather_rows: empty map");
    V1_REQUIRE(pool_rows > 0 || (int64_t)rows * top == 0, "gather_rows: empty pool");
    RowMap rm{ids, ids_stride, top, map, map_len, map_stride, map_shift, pool_rows, pool_stride_bytes, 0};
    return launch_rows(static_cast<const uint8_t*>(pool), rm, (int64_t)rows * top, row_bytes,
                       pool_rows * pool_stride_bytes, static_cast<uint8_t*>(out), as_stream(stream));
}

extern "C" int v1_gather_slots(const void* k_pool, const void* v_pool, int64_t pool_slots,
                               int32_t elem_bytes, int64_t ks0, int64_t ks1, int64_t ks2,
                               int64_t vs0, int64_t vs1, int64_t vs2, int32_t head,
                               const int32_t* req, int64_t req_len, const int32_t* ids,
                               int64_t ids_stride, int32_t rows, int32_t top, void* k_out,
                               void* v_out, void* stream) {
    V1_REQUIRE(rows >= 0 && top >= 0 && head >= 0, "gather_slots: negative shape");
    V1_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4,
               "gather_slots: unsupported element size %d", elem_bytes);
    V1_REQUIRE(req != nullptr && req_len > 0, "gather_slots: empty request map");
    const int64_t total = (int64_t)rows * top;
    if (total == 0) return V1_OK;
    hipStream_t st = as_stream(stream);
    const int dim = V1_HEAD_DIM;
    const void* pools[2] = {k_pool, v_pool};
    void* outs[2] = {k_out, v_out};
    const int64_t s0[2] = {ks0, vs0}, s1[2] = {ks1, vs1}, s2[2] = {ks2, vs2};
    for (int w = 0; w < 2; ++w) {
        RowMap rm{ids, ids_stride, top, req, req_len, 0, 0, pool_slots, 0, 0};
        const int64_t row_bytes = (int64_t)dim * elem_bytes;
        const bool fast = s2[w] == 1 && (s0[w] * elem_bytes) % 16 == 0 && (s1[w] * elem_bytes) % 16 == 0 &&
                          aligned16(pools[w]) && aligned16(outs[w]);
        int rc;
        if (fast) {
            rm.pool_stride_bytes = s0[w] * elem_bytes;
            rm.base_offset_bytes = (int64_t)head * s1[w] * elem_bytes;
            rc = launch_rows(static_cast<const uint8_t*>(pools[w]), rm, total, row_bytes, pool_slots * s0[w] * elem_bytes,
                             static_cast<uint8_t*>(outs[w]), st);
        } else {
            rm.pool_stride_bytes = s0[w];  // element units for the strided kernel
            rm.base_offset_bytes = (int64_t)head * s1[w];
            const int64_t blocks = cdiv(total * dim, kThreads);
            if (elem_bytes == 2)
                hipLaunchKernelGGL(gather_strided<uint16_t>, dim3((uint32_t)blocks), dim3(kThreads), 0, st,
                                   static_cast<const uint16_t*>(pools[w]), rm, total, s2[w], dim,
                                   static_cast<uint16_t*>(outs[w]));
            else if (elem_bytes == 4)
                hipLaunchKernelGGL(gather_strided<uint32_t>, dim3((uint32_t)blocks), dim3(kThreads), 0, st,
                                   static_cast<const uint32_t*>(pools[w]), rm, total, s2[w], dim,
                                   static_cast<uint32_t*>(outs[w]));
            else
                hipLaunchKernelGGL(gather_strided<uint8_t>, dim3((uint32_t)blocks), dim3(kThreads), 0, st,
                                   static_cast<const uint8_t*>(pools[w]), rm, total, s2[w], dim,
                                   static_cast<uint8_t*>(outs[w]));
            rc = V1_LAUNCHED("gather_strided");
        }
        if (rc != V1_OK) return rc;
    }
    return V1_OK;
}
