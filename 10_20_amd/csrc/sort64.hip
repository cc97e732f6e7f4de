// Device-wide stable LSD radix sort of (uint64 key, uint32 value) pairs,
// ascending by key; equal keys keep their input order.  Used to group page
// keys for the batched page manager (the int64 form of _sort,
// sglang/srt/layers/attention/v1_native/fused_grouping.py:64-76, over a whole
// batch instead of one 4096-key group).
//
// Each of the 8 passes (8-bit digits) runs three kernels:
//   count   one work-group per 4096-pair tile: digit histogram of the tile
//   scan    one work-group: exclusive prefix over (digit, tile), digit-major,
//           which is the first output slot of each tile's digit run
//   scatter each tile again, 256 pairs per round in input order: a pair's
//           slot = tile base of its digit + pairs of that digit in earlier
//           rounds + in earlier waves of this round + in lower lanes (lanes
//           with the same digit found with 8 ballots)
// Passes whose digit is equal for every key are skipped by the host only when
// the caller says so (`key_bits`), never by inspecting the data.
#include "common.h"

namespace v1 {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kPerThread = 16;
constexpr int kTile = kSortThreads * kPerThread;  // 4096 pairs
constexpr int kDigits = 256;

__global__ __launch_bounds__(kSortThreads) void radix_count(const uint64_t* keys, int64_t n, int shift,
                                                            uint32_t* hist, uint32_t tiles) {
    __shared__ uint32_t h[kDigits];
    const int t = threadIdx.x;
    h[t] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kTile;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int64_t k = base + i * kSortThreads + t;
        if (k < n) atomicAdd(&h[(keys[k] >> shift) & 0xff], 1u);
    }
    __syncthreads();
    hist[(int64_t)t * tiles + blockIdx.x] = h[t];
}

// Exclusive prefix over hist[0 .. 256 * tiles) in place, one work-group.
__global__ __launch_bounds__(kSortThreads) void radix_scan(uint32_t* hist, int64_t total) {
    __shared__ uint32_t red[kSortWaves];
    __shared__ uint32_t carry;
    const int t = threadIdx.x, w = t / kWave, l = __lane_id();
    if (t == 0) carry = 0;
    __syncthreads();
    for (int64_t b = 0; b < total; b += kSortThreads) {
        const int64_t i = b + t;
        const uint32_t v = i < total ? hist[i] : 0u;
        const uint32_t x = wave_inclusive_sum(v);
        if (l == kWave - 1) red[w] = x;
        __syncthreads();
        uint32_t before = carry, all = 0;
#pragma unroll
        for (int k = 0; k < kSortWaves; ++k) {
            before += k < w ? red[k] : 0u;
            all += red[k];
        }
        if (i < total) hist[i] = before + x - v;
        __syncthreads();
        if (t == 0) carry += all;
        __syncthreads();
    }
}

__global__ __launch_bounds__(kSortThreads) void radix_scatter(const uint64_t* keys_in, const uint32_t* vals_in,
                                                              uint64_t* keys_out, uint32_t* vals_out, int64_t n,
                                                              int shift, const uint32_t* hist, uint32_t tiles) {
    __shared__ uint32_t base[kDigits];               // next slot of each digit
    __shared__ uint32_t wave_cnt[kSortWaves][kDigits];  // this round's count per wave
    const int t = threadIdx.x, w = t / kWave, l = __lane_id();
    base[t] = hist[(int64_t)t * tiles + blockIdx.x];
    const int64_t tile0 = (int64_t)blockIdx.x * kTile;
    for (int r = 0; r < kPerThread; ++r) {
        const int64_t k = tile0 + (int64_t)r * kSortThreads + t;
        const bool ok = k < n;
        const uint64_t key = ok ? keys_in[k] : 0ull;
        const uint32_t val = ok ? vals_in[k] : 0u;
        const uint32_t d = (uint32_t)(key >> shift) & 0xff;
        // lanes of this wave holding the same digit
        uint64_t peers = __ballot(ok);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t m = __ballot((d >> b) & 1);
            peers &= ((d >> b) & 1) ? m : ~m;
        }
        const uint32_t below = (uint32_t)__popcll(peers & ((1ull << l) - 1ull));
        const bool leader = ok && below == 0;
#pragma unroll
        for (int i = 0; i < kSortWaves; ++i) wave_cnt[i][t] = 0;
        __syncthreads();
        if (leader) wave_cnt[w][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        if (ok) {
            uint32_t slot = base[d] + below;
            for (int i = 0; i < w; ++i) slot += wave_cnt[i][d];
            keys_out[slot] = key;
            vals_out[slot] = val;
        }
        __syncthreads();
        uint32_t round = 0;
#pragma unroll
        for (int i = 0; i < kSortWaves; ++i) round += wave_cnt[i][t];
        base[t] += round;
        __syncthreads();
    }
}

}  // namespace

int64_t sort_pairs_workspace(int64_t n) {
    const int64_t tiles = cdiv(std::max<int64_t>(n, 1), kTile);
    return n * (8 + 4) + tiles * kDigits * 4 + 256;
}

// Sorts n pairs from (keys, vals) into (keys_out, vals_out); the workspace
// holds a second buffer and the histograms.  key_bits: the low bits that can
// differ (64 for arbitrary keys); passes above it are skipped.
int sort_pairs(const uint64_t* keys, const uint32_t* vals, uint64_t* keys_out, uint32_t* vals_out, int64_t n,
               int key_bits, void* ws, int64_t ws_bytes, hipStream_t st, const char* name) {
    V1_REQUIRE(n >= 0 && n < (1ll << 31), "%s: bad pair count", name);
    if (n == 0) return V1_OK;
    V1_REQUIRE(ws != nullptr && ws_bytes >= sort_pairs_workspace(n), "%s: sort workspace of %lld bytes required",
               name, (long long)sort_pairs_workspace(n));
    const uint32_t tiles = (uint32_t)cdiv(n, kTile);
    uint64_t* k2 = static_cast<uint64_t*>(ws);
    uint32_t* v2 = reinterpret_cast<uint32_t*>(k2 + n);
    uint32_t* hist = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(ws) + n * 12 + 128);
    hist = reinterpret_cast<uint32_t*>((reinterpret_cast<uintptr_t>(hist) + 127) & ~uintptr_t(127));
    const int passes = (std::max(1, std::min(key_bits, 64)) + 7) / 8;
    // pass p reads src, writes dst; the last pass writes the output
    const uint64_t* sk = keys;
    const uint32_t* sv = vals;
    for (int p = 0; p < passes; ++p) {
        // final pass lands in the output buffer
        const bool last = p == passes - 1;
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        uint64_t* dk = to_out ? keys_out : k2;
        uint32_t* dv = to_out ? vals_out : v2;
        (void)last;
        hipLaunchKernelGGL(radix_count, dim3(tiles), dim3(kSortThreads), 0, st, sk, n, 8 * p, hist, tiles);
        int rc = V1_LAUNCHED(name);
        if (rc != V1_OK) return rc;
        hipLaunchKernelGGL(radix_scan, dim3(1), dim3(kSortThreads), 0, st, hist, (int64_t)tiles * kDigits);
        rc = V1_LAUNCHED(name);
        if (rc != V1_OK) return rc;
        hipLaunchKernelGGL(radix_scatter, dim3(tiles), dim3(kSortThreads), 0, st, sk, sv, dk, dv, n, 8 * p, hist,
                           tiles);
        rc = V1_LAUNCHED(name);
        if (rc != V1_OK) return rc;
        sk = dk;
        sv = dv;
    }
    return V1_OK;
}

}  // namespace v1

using namespace v1;

extern "C" int64_t v1_sort_pairs_u64_workspace(int64_t n) { return n < 0 ? 0 : sort_pairs_workspace(n); }

extern "C" int v1_sort_pairs_u64(const uint64_t* keys, const uint32_t* vals, uint64_t* keys_out, uint32_t* vals_out,
                                 int64_t n, int32_t key_bits, void* workspace, int64_t workspace_bytes, void* stream) {
    V1_REQUIRE(key_bits >= 1 && key_bits <= 64, "sort_pairs_u64: key_bits must be in [1, 64]");
    V1_REQUIRE(n == 0 || (keys != nullptr && vals != nullptr && keys_out != nullptr && vals_out != nullptr),
               "sort_pairs_u64: null buffer");
    V1_REQUIRE(keys_out != keys && vals_out != vals, "sort_pairs_u64: output must not alias the input");
    return sort_pairs(keys, vals, keys_out, vals_out, n, key_bits, workspace, workspace_bytes, as_stream(stream),
                      "sort_pairs_u64");
}

// ------------------------------------------------------------------ scan
// Exclusive prefix sum over n uint32 in three launches: per-tile scans with
// tile totals, one work-group over the totals, then the tile offsets added.
namespace v1 {
namespace {

__device__ __forceinline__ uint32_t block_exclusive(uint32_t v, uint32_t (&red)[kSortWaves], uint32_t& all) {
    const int t = threadIdx.x, w = t / kWave, l = __lane_id();
    const uint32_t x = wave_inclusive_sum(v);
    if (l == kWave - 1) red[w] = x;
    __syncthreads();
    uint32_t before = 0;
    all = 0;
#pragma unroll
    for (int k = 0; k < kSortWaves; ++k) {
        before += k < w ? red[k] : 0u;
        all += red[k];
    }
    __syncthreads();
    return before + x - v;
}

// thread t owns kPerThread consecutive elements of the tile
__global__ __launch_bounds__(kSortThreads) void scan_tiles(const uint32_t* in, uint32_t* out, int64_t n,
                                                           uint32_t* tile_sum) {
    __shared__ uint32_t red[kSortWaves];
    const int t = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * kTile + (int64_t)t * kPerThread;
    uint32_t v[kPerThread];
    uint32_t local = 0;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        v[i] = base + i < n ? in[base + i] : 0u;
        local += v[i];
    }
    uint32_t all;
    uint32_t run = block_exclusive(local, red, all);
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        if (base + i < n) out[base + i] = run;
        run += v[i];
    }
    if (t == 0) tile_sum[blockIdx.x] = all;
}

__global__ __launch_bounds__(kSortThreads) void scan_sums(uint32_t* tile_sum, int64_t tiles, uint32_t* total) {
    __shared__ uint32_t red[kSortWaves];
    __shared__ uint32_t carry;
    const int t = threadIdx.x;
    if (t == 0) carry = 0;
    __syncthreads();
    for (int64_t b = 0; b < tiles; b += kSortThreads) {
        const uint32_t v = b + t < tiles ? tile_sum[b + t] : 0u;
        uint32_t all;
        const uint32_t ex = block_exclusive(v, red, all);
        if (b + t < tiles) tile_sum[b + t] = carry + ex;
        __syncthreads();
        if (t == 0) carry += all;
        __syncthreads();
    }
    if (t == 0) *total = carry;
}

__global__ __launch_bounds__(kSortThreads) void scan_add(uint32_t* out, int64_t n, const uint32_t* tile_sum) {
    const int64_t base = (int64_t)blockIdx.x * kTile;
    const uint32_t add = tile_sum[blockIdx.x];
    for (int i = threadIdx.x; i < kTile; i += kSortThreads)
        if (base + i < n) out[base + i] += add;
}

}  // namespace

int64_t scan_workspace(int64_t n) { return (cdiv(std::max<int64_t>(n, 1), kTile) + 64) * 4; }

int scan_exclusive(const uint32_t* in, uint32_t* out, uint32_t* total, int64_t n, void* ws, int64_t ws_bytes,
                   hipStream_t st, const char* name) {
    V1_REQUIRE(n >= 0 && n < (1ll << 31), "%s: bad scan length", name);
    V1_REQUIRE(ws != nullptr && ws_bytes >= scan_workspace(n), "%s: scan workspace too small", name);
    const int64_t tiles = cdiv(std::max<int64_t>(n, 1), kTile);
    uint32_t* sums = static_cast<uint32_t*>(ws);
    hipLaunchKernelGGL(scan_tiles, dim3((uint32_t)tiles), dim3(kSortThreads), 0, st, in, out, n, sums);
    int rc = V1_LAUNCHED(name);
    if (rc != V1_OK) return rc;
    hipLaunchKernelGGL(scan_sums, dim3(1), dim3(kSortThreads), 0, st, sums, tiles, total);
    rc = V1_LAUNCHED(name);
    if (rc != V1_OK) return rc;
    hipLaunchKernelGGL(scan_add, dim3((uint32_t)tiles), dim3(kSortThreads), 0, st, out, n, sums);
    return V1_LAUNCHED(name);
}

}  // namespace v1
