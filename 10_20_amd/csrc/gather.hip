// Slot gather: copies one source row per (query row, top slot) into a dense
// workspace, zero-filling padding ids.  Pure HBM work: each work-group first
// maps its tile of slots to source byte offsets in LDS (one id / map lookup
// per slot), then copies the tile as 16-byte chunks in one pass: every lane
// issues all of its loads, then all of its stores, and exits.  Both the
// workspace writes and the per-row reads are fully coalesced.  Workspace
// stores are non-temporal: the workspace is written once per call and read by
// the attention consumer.
//
// Semantics follow sglang/srt/layers/attention/v1_native/kernels.py:62-77.
#include "common.h"

namespace v1 {
namespace {

constexpr int kThreads = 256;
// Copy shapes, measured on MI355X with 656-byte rows (41 chunks) and
// 1024 x 2048 or 4096 x 2048 slots.  A tile is the largest power of two of
// slots whose chunks fit one pass of kThr x kUnroll loads; tiles that are not
// a power of two end mid-row on the XCDs' round-robin and take 1.2-1.8x as
// long.  A small pool (at most 64 MB) stays cache-resident and the workspace
// writes set the pace: 1024 threads x 11 loads (256-slot tiles, two
// work-groups per CU) copy 4096 x 2048 rows of a 21.5 MB pool in 0.88 ms,
// against 0.96-0.98 ms for 512-slot tiles (21 loads, or 8 loads over three
// passes), 0.93 ms for 128-slot tiles and 1.04-1.06 ms for 64-slot ones.  A
// pool well above the caches streams from HBM and favours short tiles:
// 512 threads x 6 loads (64-slot tiles) copy 1024 x 2048 rows of a 688 MB
// pool in 410 us, against 412-418 us for 128- and 256-slot tiles.
constexpr int kThreadsCached = 1024, kUnrollCached = 11;
constexpr int kThreadsStream = 512, kUnrollStream = 6;
constexpr int kMaxTile = 1024;  // LDS offsets per work-group
constexpr int64_t kCachedPoolBytes = 64ll << 20;
// Word 3 of a raw buffer descriptor (stride 0, 32-bit dwords): stores at byte
// offsets at or past the descriptor's length are dropped.
constexpr int32_t kRawDword = 0x00020000;
constexpr int kNonTemporal = 2;  // buffer store cache policy: nt

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

// Copies the (1 << tile_shift)-slot tile blockIdx.x of `chunks` 16-byte
// chunks per slot into the dense workspace `out`.  The copy has no branches:
// lanes of padding slots, and lanes past the tile's last chunk, load the
// pool's first chunk and zero it, and the stores go through a descriptor
// that ends at the tile's last byte, so the hardware drops those past it.
// Without branches the compiler waits for each load just before its store;
// with per-lane conditions around loads and stores it waited for every
// outstanding store before issuing the next loads.  `pool` must hold at
// least one row.
template <int kThr, int kUnroll>
__global__ __launch_bounds__(kThr) void gather_rows16(
    const uint8_t* __restrict__ pool, RowMap rm, int64_t total_slots, int32_t chunks,
    uint32_t chunk_magic, int32_t tile_shift, uint8_t* __restrict__ out) {
    __shared__ int64_t src[kMaxTile];
    const int tile = 1 << tile_shift;
    const int64_t first = (int64_t)blockIdx.x << tile_shift;
    const int tid = threadIdx.x;
    for (int s = tid; s < tile; s += kThr) {
        const int64_t t = first + s;
        src[s] = t < total_slots ? rm(t) : -1;
    }
    __syncthreads();
    const int64_t left = total_slots - first;
    const int slots = left < tile ? (int)left : tile;
    const uint32_t n = (uint32_t)slots * (uint32_t)chunks;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(out + first * (int64_t)chunks * 16, 0, (int32_t)(n * 16u),
                                                      kRawDword);
    for (uint32_t base = 0; base < n; base += kThr * kUnroll) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t g = base + u * kThr + tid;
            uint32_t sl = chunks == 1 ? g : small_div(g, chunk_magic);
            sl = sl < (uint32_t)slots ? sl : (uint32_t)(slots - 1);
            const uint32_t c = g - sl * (uint32_t)chunks;
            const int64_t off = src[sl];
            const bool ok = off >= 0 && g < n;
            v[u] = *reinterpret_cast<const u32x4*>(ok ? pool + off + (int64_t)c * 16 : pool);
            if (!ok) v[u] = u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            __builtin_amdgcn_raw_buffer_store_b128(v[u], rs, (int32_t)((base + u * kThr + tid) * 16u), 0, kNonTemporal);
    }
}

// Largest power-of-two tile (log2) whose chunks fit one pass of `per_pass`.
int tile_shift_for(int32_t chunks, int per_pass) {
    int shift = 0;
    while ((1 << (shift + 1)) <= kMaxTile && (int64_t)chunks << (shift + 1) <= per_pass) ++shift;
    return shift;
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

// pool_bytes: the bytes of the pool the copy can read (0: an empty pool);
// it picks the copy shape.
int launch_rows(const uint8_t* pool, const RowMap& rm, int64_t total, int64_t row_bytes, int64_t pool_bytes,
                uint8_t* out, hipStream_t st) {
    if (total == 0) return V1_OK;
    const int32_t chunks = (int32_t)(row_bytes / 16);
    if (pool_bytes == 0) {
        // every slot is a padding slot: zero rows, with no pool row to load
        hipLaunchKernelGGL(gather_strided<uint8_t>, dim3((uint32_t)cdiv(total * row_bytes, kThreads)), dim3(kThreads), 0,
                           st, pool, rm, total, (int64_t)1, (int32_t)row_bytes, out);
        return V1_LAUNCHED("gather_strided");
    }
    const uint32_t magic = chunks == 1 ? 0u : small_div_magic((uint32_t)chunks);
    // The copy is write-bound, and takes the cached shape, when the pool
    // stays in the caches or when it writes every pool byte four or more
    // times on average (1024 x 2048 rows drawn from 2688 candidates of a
    // 172 MB pool: 214 us against 254 us with the streamed shape).
    const bool cached = pool_bytes <= kCachedPoolBytes || total * row_bytes >= 4 * pool_bytes;
    if (!cached) {
        const int shift = tile_shift_for(chunks, kThreadsStream * kUnrollStream);
        hipLaunchKernelGGL((gather_rows16<kThreadsStream, kUnrollStream>), dim3((uint32_t)cdiv(total, 1ll << shift)),
                           dim3(kThreadsStream), 0, st, pool, rm, total, chunks, magic, shift, out);
    } else {
        const int shift = tile_shift_for(chunks, kThreadsCached * kUnrollCached);
        hipLaunchKernelGGL((gather_rows16<kThreadsCached, kUnrollCached>), dim3((uint32_t)cdiv(total, 1ll << shift)),
                           dim3(kThreadsCached), 0, st, pool, rm, total, chunks, magic, shift, out);
    }
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
            // (the copy reads one head's row of each slot: pool_slots rows of
            // row_bytes, whatever the slot stride)
            rc = launch_rows(static_cast<const uint8_t*>(pools[w]), rm, total, row_bytes, pool_slots * row_bytes,
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
