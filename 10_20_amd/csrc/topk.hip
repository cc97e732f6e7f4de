// Exact Top-T (T <= 2048) over fp32 score rows, with the V1 sink/tail mask and
// raw -> logical -> physical epilogue (fused.topk) or the page-table transform
// epilogue (topk_transform_512_v2), plus the unfused mask_fine / output_ids.
//
// Selection contract: the T largest scores of a row, ties toward the lower
// candidate index, -0.0 == +0.0; each output row lists the chosen candidates
// in ascending index order followed by -1 padding.  Rows of at most T
// candidates take every candidate (sglang/kernels/jit/csrc/deepseek_v4/
// topk_v2.cuh:136-143).
//
// Design (one 1024-thread work-group per row, wave64):
//  * the row is loaded once, as order-preserving uint32 keys, into registers
//    (striped float4 loads: element j = c*4096 + 4*t + e);
//  * three LDS radix-histogram passes (12/10/10 bits) locate the T-th largest
//    key `tau` and how many tau-valued elements must be taken (`r`);
//  * one block-wide packed (greater | equal << 16) prefix scan in index order
//    gives every chosen element its output slot: gt_before + min(eq_before, r).
//    The output is therefore ascending and deterministic without a sort.
// Rows longer than 32768 columns are cut into 32768-column segments: one
// work-group selects each segment's Top-T into a workspace (ascending index),
// and a merge work-group selects the row's Top-T from the concatenation.
#include "common.h"

namespace v1 {
namespace {

constexpr int kBlock = 1024;
constexpr int kWaves = kBlock / kWave;  // 16
constexpr int kChunk = 4 * kBlock;      // elements per striped chunk
constexpr int kSegment = 32768;         // columns per work-group
constexpr uint32_t kNegInfKey = 0x007fffffu;
constexpr uint32_t kInfBit = 0x80000000u;

struct SelSmem {
    uint32_t hist[4096];
    uint32_t wtot[kWaves];
    uint32_t ctot[8 * kWaves];
    uint32_t cbase[8 * kWaves];
    uint32_t bc[2];
    int32_t sel[V1_MAX_TOPK];  // chosen positions (| kInfBit when the score is -inf)
    int32_t maskpage[512];     // V1 mask: page per selected rank, -1 when unmasked
};

__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, SelSmem& sm) {
    const int w = threadIdx.x / kWave;
    const uint32_t x = wave_inclusive_sum(v);
    if (__lane_id() == kWave - 1) sm.wtot[w] = x;
    __syncthreads();
    uint32_t base = 0;
    for (int k = 0; k < w; ++k) base += sm.wtot[k];
    return base + x;
}

// One radix pass: histogram the digit (key >> SHIFT) & (BINS-1) of every key
// matching `prefix` under `pmask`, then locate the bin holding the
// `remaining`-th largest such key.
template <int ITEMS, int BINS, int SHIFT>
__device__ __forceinline__ void radix_pass(const uint32_t (&key)[ITEMS], uint32_t& prefix,
                                           uint32_t& pmask, uint32_t& remaining, SelSmem& sm) {
    const int t = threadIdx.x;
    for (int i = t; i < BINS; i += kBlock) sm.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
        const uint32_t k = key[i];
        if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> SHIFT) & (BINS - 1)], 1u);
    }
    __syncthreads();
    constexpr int BPT = BINS / kBlock;
    uint32_t h[BPT];
    uint32_t local = 0;
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
        h[b] = sm.hist[BINS - 1 - (BPT * t + b)];
        local += h[b];
    }
    const uint32_t incl = block_incl_scan(local, sm);
    const uint32_t excl = incl - local;
    if (excl < remaining && remaining <= incl) {
        uint32_t acc = excl;
#pragma unroll
        for (int b = 0; b < BPT; ++b) {
            if (acc + h[b] >= remaining) {
                sm.bc[0] = BINS - 1 - (BPT * t + b);
                sm.bc[1] = acc;
                break;
            }
            acc += h[b];
        }
    }
    __syncthreads();
    remaining -= sm.bc[1];
    prefix |= sm.bc[0] << SHIFT;
    pmask |= (uint32_t)(BINS - 1) << SHIFT;
}

// Selects the T largest keys (ties -> lower position) of a register tile and
// writes their positions, ascending, to sm.sel[0..T) and their keys to
// sm.hist[0..T) (the histogram is free once the radix passes are done).
// Requires more than T keys above the padding key 0.  Position of item i of
// thread t: (i/4)*kChunk + 4*t + i%4.  Ends with a barrier.
template <int ITEMS>
__device__ void select_top(const uint32_t (&key)[ITEMS], uint32_t T, SelSmem& sm) {
    uint32_t prefix = 0, pmask = 0, remaining = T;
    radix_pass<ITEMS, 4096, 20>(key, prefix, pmask, remaining, sm);
    radix_pass<ITEMS, 1024, 10>(key, prefix, pmask, remaining, sm);
    radix_pass<ITEMS, 1024, 0>(key, prefix, pmask, remaining, sm);
    const uint32_t tau = prefix, r = remaining;

    constexpr int NC = ITEMS / 4;
    const int t = threadIdx.x, w = t / kWave, lane = __lane_id();
    uint32_t cnt[NC], incl[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        uint32_t n = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t k = key[4 * c + e];
            n += k > tau ? 1u : (k == tau ? 0x10000u : 0u);
        }
        cnt[c] = n;
        incl[c] = wave_inclusive_sum(n);
    }
    if (lane == kWave - 1) {
#pragma unroll
        for (int c = 0; c < NC; ++c) sm.ctot[c * kWaves + w] = incl[c];
    }
    __syncthreads();
    if (w == 0) {
        // exclusive scan over (chunk, wave) in index order; 2 entries per lane
        const int q0 = 2 * lane, q1 = 2 * lane + 1;
        const uint32_t a = q0 < NC * kWaves ? sm.ctot[q0] : 0u;
        const uint32_t b = q1 < NC * kWaves ? sm.ctot[q1] : 0u;
        const uint32_t s = wave_inclusive_sum(a + b);
        if (q0 < NC * kWaves) sm.cbase[q0] = s - a - b;
        if (q1 < NC * kWaves) sm.cbase[q1] = s - b;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t before = sm.cbase[c * kWaves + w] + incl[c] - cnt[c];
        uint32_t gt = before & 0xffffu, eq = before >> 16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t k = key[4 * c + e];
            const int32_t j = c * kChunk + 4 * t + e;
            const int32_t tag = k == kNegInfKey ? (int32_t)kInfBit : 0;
            if (k > tau) {
                const uint32_t at = gt + min(eq, r);
                sm.sel[at] = j | tag;
                sm.hist[at] = k;
                ++gt;
            } else if (k == tau) {
                if (eq < r) {
                    sm.sel[gt + eq] = j | tag;
                    sm.hist[gt + eq] = k;
                }
                ++eq;
            }
        }
    }
    __syncthreads();
}

// Loads columns [0, n) of one row (n <= ITEMS*1024) as keys; others get key 0.
template <int ITEMS>
__device__ __forceinline__ void load_keys(const float* __restrict__ rowp, int32_t n, uint32_t (&key)[ITEMS]) {
    constexpr int NC = ITEMS / 4;
    const int t = threadIdx.x;
    const bool vec = (reinterpret_cast<uintptr_t>(rowp) & 15) == 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int32_t j = c * kChunk + 4 * t;
        if (vec && j + 3 < n) {
            const float4 v = *reinterpret_cast<const float4*>(rowp + j);
            key[4 * c + 0] = score_key(v.x);
            key[4 * c + 1] = score_key(v.y);
            key[4 * c + 2] = score_key(v.z);
            key[4 * c + 3] = score_key(v.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) key[4 * c + e] = j + e < n ? score_key(rowp[j + e]) : 0u;
        }
    }
}

// ------------------------------------------------------------------ V1 map
struct V1Params {
    float* scores;
    int64_t score_stride;
    int32_t cols;
    const int32_t* fine_lens;
    const int32_t* members;
    int64_t member_pages;
    const int32_t* rt;
    const int32_t* nt;
    int32_t pages;
    const void* selected;
    int32_t sel64;
    int32_t take_stride;
    const int32_t* lens;
    const int32_t* takes;
    int32_t* physical;
    int32_t* logical;
    int32_t* raw;
    int32_t topk;
    int32_t window;
    int32_t mask;
    int32_t* expanded;
    int32_t expansion_stride;
    int32_t physical_output;
    int32_t bucket_from_rank;
    const int32_t* fine_table;
    int32_t fine_table_cols;
    int32_t direct_fine;
};

struct RowInfo {
    int32_t n, take, sink, tail;
};

__device__ __forceinline__ RowInfo v1_row_info(const V1Params& p, int64_t row) {
    RowInfo ri;
    ri.n = p.lens[row];
    ri.take = p.takes[row];
    ri.sink = min(ri.n, 64);
    ri.tail = max(ri.sink, min(max(ri.n - 1, 0) / 1024 * 1024, max(ri.sink, ri.n - p.window)));
    // Memory-safety clamps: a take beyond the selected / fine-table row is out of contract.
    ri.take = max(0, min(ri.take, p.take_stride));
    if (p.direct_fine) ri.take = min(ri.take, p.fine_table_cols);
    return ri;
}

__device__ __forceinline__ int32_t sel_rank(const V1Params& p, int64_t row, int32_t r) {
    return p.sel64 ? (int32_t) static_cast<const int64_t*>(p.selected)[row * p.take_stride + r]
                   : static_cast<const int32_t*>(p.selected)[row * p.take_stride + r];
}

// Page whose members must be masked for selected rank r, or -1.
// sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:71-107.
__device__ __forceinline__ int32_t v1_mask_page(const V1Params& p, int64_t row, int32_t r, const RowInfo& ri) {
    const int32_t rank = sel_rank(p, row, r);
    if (rank < 0 || rank >= p.pages) return -1;
    int32_t page = p.rt[row * p.pages + rank];
    int32_t bucket;
    if (p.bucket_from_rank) {
        bucket = (rank / 16) * 1024;
    } else {
        if (page < 0 || page >= p.member_pages) return -1;
        bucket = (p.members[(int64_t)page * 64] / 1024) * 1024;
    }
    if (!(bucket < ri.sink || bucket + 1024 > ri.tail)) return -1;
    if (page < 0 || page >= p.member_pages) return -1;
    return page;
}

// Applies the sink/tail mask to columns [lo, hi) of the row: writes -inf in
// place and, for columns held in registers, turns their key into the -inf key.
template <int ITEMS>
__device__ void v1_apply_mask(const V1Params& p, int64_t row, const RowInfo& ri, int32_t lo, int32_t hi,
                              uint32_t (&key)[ITEMS], int32_t reg_n, SelSmem& sm) {
    const int t = threadIdx.x;
    const int32_t limit = min(hi, min(ri.take * 64, p.cols));
    const int32_t r0 = lo / 64, r1 = limit > lo ? (limit + 63) / 64 : r0;  // ranks touching [lo, limit)
    for (int32_t r = r0 + t; r < r1; r += kBlock) sm.maskpage[r - r0] = v1_mask_page(p, row, r, ri);
    __syncthreads();
    float* rowp = p.scores + row * p.score_stride;
    constexpr int NC = ITEMS / 4;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int32_t jl = c * kChunk + 4 * t + e;  // position inside the tile
            const int32_t j = lo + jl;
            if (j < limit) {
                const int32_t page = sm.maskpage[j / 64 - r0];
                if (page >= 0) {
                    const int32_t lg = p.members[(int64_t)page * 64 + (j & 63)];
                    if (lg < ri.sink || lg >= ri.tail) {
                        rowp[j] = -__builtin_huge_valf();
                        if (jl < reg_n) key[4 * c + e] = kNegInfKey;
                    }
                }
            }
        }
    }
    __syncthreads();
}

// raw -> logical -> physical for one output slot.
// sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:121-148.
__device__ __forceinline__ void v1_emit(const V1Params& p, int64_t row, const RowInfo& ri, int32_t tx,
                                        int32_t raw, bool neg_inf) {
    int32_t logical = -1, physical = -1;
    if (raw >= 0 && !neg_inf) {
        if (raw < ri.take * 64) {
            int32_t page = -1;
            if (p.direct_fine) {
                page = p.fine_table[row * p.fine_table_cols + raw / 64];
            } else {
                const int32_t rank = sel_rank(p, row, raw / 64);
                if (rank >= 0 && rank < p.pages) page = p.rt[row * p.pages + rank];
            }
            if (page >= 0 && page < p.member_pages) logical = p.members[(int64_t)page * 64 + (raw & 63)];
        } else {
            const int32_t off = raw - ri.take * 64;
            logical = off < ri.sink ? off : ri.tail + off - ri.sink;
        }
        if (logical >= 0 && logical < ri.n && logical / 64 < p.pages) {
            physical = p.nt[row * p.pages + logical / 64] * 64 + (logical & 63);
        } else {
            logical = -1;
        }
    }
    const int64_t dst = row * p.topk + tx;
    p.logical[dst] = logical;
    if (p.physical_output) {
        p.physical[dst] = physical;
        p.raw[dst] = raw;
    }
    if (p.expansion_stride) {
        const int32_t b = logical * 4;
        int4 v = logical < 0 ? make_int4(-1, -1, -1, -1) : make_int4(b, b + 1, b + 2, b + 3);
        *reinterpret_cast<int4*>(p.expanded + row * p.expansion_stride + 4 * tx) = v;
    }
}

__device__ __forceinline__ void v1_pad_expansion(const V1Params& p, int64_t row) {
    if (p.expansion_stride)
        for (int j = p.topk * 4 + threadIdx.x; j < p.expansion_stride; j += kBlock)
            p.expanded[row * p.expansion_stride + j] = -1;
}

// ---------------------------------------------------------- transform map
struct TransformParams {
    const float* scores;
    int64_t score_stride;
    int32_t cols;
    const int32_t* seq_lens;
    const int32_t* page_table;
    int64_t page_table_stride;
    int32_t page_table_cols;
    int32_t page_bits;
    int32_t* page_indices;
    int32_t* raw_indices;
    int32_t topk;
};

__device__ __forceinline__ void transform_emit(const TransformParams& p, int64_t row, int32_t tx, int32_t raw) {
    int32_t out = -1;
    if (raw >= 0) {
        const int32_t e = raw >> p.page_bits;
        if (e < p.page_table_cols)
            out = (p.page_table[row * p.page_table_stride + e] << p.page_bits) | (raw & ((1 << p.page_bits) - 1));
    }
    const int64_t dst = row * p.topk + tx;
    p.page_indices[dst] = out;
    if (p.raw_indices) p.raw_indices[dst] = raw;
}

// --------------------------------------------------------- single pass
template <int ITEMS>
__global__ __launch_bounds__(kBlock) void v1_topk_rows(V1Params p) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const RowInfo ri = v1_row_info(p, row);
    const int32_t L = max(0, min(p.fine_lens[row], p.cols));
    uint32_t key[ITEMS];
    load_keys<ITEMS>(p.scores + row * p.score_stride, L, key);
    if (p.mask) v1_apply_mask<ITEMS>(p, row, ri, 0, p.cols, key, L, sm);
    const int32_t T = p.topk;
    int32_t nsel;
    if (L <= T) {
        // every candidate; -inf status needs the key of position tx
        constexpr int NC = ITEMS / 4;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t j = c * kChunk + 4 * threadIdx.x + e;
                if (j < L) sm.sel[j] = j | (key[4 * c + e] == kNegInfKey ? (int32_t)kInfBit : 0);
            }
        __syncthreads();
        nsel = L;
    } else {
        select_top<ITEMS>(key, (uint32_t)T, sm);
        nsel = T;
    }
    for (int tx = threadIdx.x; tx < T; tx += kBlock) {
        const int32_t s = tx < nsel ? sm.sel[tx] : -1;
        const bool inf = s != -1 && (s & (int32_t)kInfBit);
        v1_emit(p, row, ri, tx, s == -1 ? -1 : (s & 0x7fffffff), inf);
    }
    v1_pad_expansion(p, row);
}

template <int ITEMS>
__global__ __launch_bounds__(kBlock) void transform_rows(TransformParams p) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    const int32_t T = p.topk;
    if (L <= T) {
        for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, tx < L ? tx : -1);
        return;
    }
    uint32_t key[ITEMS];
    load_keys<ITEMS>(p.scores + row * p.score_stride, L, key);
    select_top<ITEMS>(key, (uint32_t)T, sm);
    for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, sm.sel[tx] & 0x7fffffff);
}

// ------------------------------------------------------- segmented rows
// Workspace per (row, segment): T keys, T positions, then one count per pair.
struct Workspace {
    uint32_t* keys;
    int32_t* pos;
    int32_t* count;
    int32_t nseg;
    int32_t T;
    __device__ __forceinline__ int64_t at(int64_t row, int32_t s) const { return (row * nseg + s) * (int64_t)T; }
};

inline int64_t workspace_bytes(int32_t batch, int32_t cols, int32_t topk) {
    const int64_t nseg = cdiv(cols, kSegment);
    return (int64_t)batch * nseg * ((int64_t)topk * 8 + 4);
}

inline Workspace make_workspace(void* base, int32_t batch, int32_t cols, int32_t topk) {
    Workspace ws;
    ws.nseg = (int32_t)cdiv(cols, kSegment);
    ws.T = topk;
    const int64_t pairs = (int64_t)batch * ws.nseg;
    ws.keys = static_cast<uint32_t*>(base);
    ws.pos = reinterpret_cast<int32_t*>(ws.keys + pairs * topk);
    ws.count = ws.pos + pairs * topk;
    return ws;
}

// Segment s of a row: the segment's Top-T (all of it when shorter) into the
// workspace in ascending position.  Keys are forced >= 1 so that the merge's
// padding key 0 stays strictly below every real candidate.
__device__ void segment_select(const uint32_t (&key)[32], int32_t n, int32_t lo, int32_t T, const Workspace& ws,
                               int64_t row, int32_t s, SelSmem& sm) {
    const int64_t at = ws.at(row, s);
    if (n <= T) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t j = c * kChunk + 4 * threadIdx.x + e;
                if (j < n) {
                    ws.keys[at + j] = max(key[4 * c + e], 1u);
                    ws.pos[at + j] = lo + j;
                }
            }
        if (threadIdx.x == 0) ws.count[row * ws.nseg + s] = max(n, 0);
        return;
    }
    select_top<32>(key, (uint32_t)T, sm);
    for (int tx = threadIdx.x; tx < T; tx += kBlock) {
        ws.keys[at + tx] = max(sm.hist[tx], 1u);
        ws.pos[at + tx] = lo + (sm.sel[tx] & 0x7fffffff);
    }
    if (threadIdx.x == 0) ws.count[row * ws.nseg + s] = T;
}

__global__ __launch_bounds__(kBlock) void v1_topk_segments(V1Params p, Workspace ws) {
    __shared__ SelSmem sm;
    const int32_t s = blockIdx.x;
    const int64_t row = blockIdx.y;
    const RowInfo ri = v1_row_info(p, row);
    const int32_t L = max(0, min(p.fine_lens[row], p.cols));
    const int32_t lo = s * kSegment;
    const int32_t n = max(0, min(L - lo, kSegment));
    uint32_t key[32];
    load_keys<32>(p.scores + row * p.score_stride + lo, n, key);
    if (p.mask) v1_apply_mask<32>(p, row, ri, lo, lo + kSegment, key, n, sm);
    if (L <= p.topk) return;  // the merge kernel takes every candidate
    segment_select(key, n, lo, p.topk, ws, row, s, sm);
}

__global__ __launch_bounds__(kBlock) void transform_segments(TransformParams p, Workspace ws) {
    __shared__ SelSmem sm;
    const int32_t s = blockIdx.x;
    const int64_t row = blockIdx.y;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    if (L <= p.topk) return;
    const int32_t lo = s * kSegment;
    const int32_t n = max(0, min(L - lo, kSegment));
    uint32_t key[32];
    load_keys<32>(p.scores + row * p.score_stride + lo, n, key);
    segment_select(key, n, lo, p.topk, ws, row, s, sm);
}

// Loads the concatenated segment candidates of a row: position q = s*T + k.
template <int ITEMS>
__device__ __forceinline__ void load_candidates(const Workspace& ws, int64_t row, uint32_t (&key)[ITEMS]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < ITEMS / 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int32_t q = c * kChunk + 4 * t + e;
            const int32_t s = q / ws.T, k = q - s * ws.T;
            uint32_t v = 0u;
            if (s < ws.nseg && k < ws.count[row * ws.nseg + s]) v = ws.keys[ws.at(row, s) + k];
            key[4 * c + e] = v;
        }
}

__device__ __forceinline__ int32_t candidate_pos(const Workspace& ws, int64_t row, int32_t q) {
    const int32_t s = q / ws.T, k = q - s * ws.T;
    return ws.pos[ws.at(row, s) + k];
}

template <int ITEMS>
__global__ __launch_bounds__(kBlock) void v1_topk_merge(V1Params p, Workspace ws) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const RowInfo ri = v1_row_info(p, row);
    const int32_t L = max(0, min(p.fine_lens[row], p.cols));
    const int32_t T = p.topk;
    if (L <= T) {
        const float* rowp = p.scores + row * p.score_stride;  // already masked by the segment pass
        for (int tx = threadIdx.x; tx < T; tx += kBlock) {
            const bool ok = tx < L;
            const bool inf = ok && score_key(rowp[tx]) == kNegInfKey;
            v1_emit(p, row, ri, tx, ok ? tx : -1, inf);
        }
    } else {
        uint32_t key[ITEMS];
        load_candidates<ITEMS>(ws, row, key);
        select_top<ITEMS>(key, (uint32_t)T, sm);
        for (int tx = threadIdx.x; tx < T; tx += kBlock) {
            const int32_t q = sm.sel[tx];
            v1_emit(p, row, ri, tx, candidate_pos(ws, row, q & 0x7fffffff), (q & (int32_t)kInfBit) != 0);
        }
    }
    v1_pad_expansion(p, row);
}

template <int ITEMS>
__global__ __launch_bounds__(kBlock) void transform_merge(TransformParams p, Workspace ws) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    const int32_t T = p.topk;
    if (L <= T) {
        for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, tx < L ? tx : -1);
        return;
    }
    uint32_t key[ITEMS];
    load_candidates<ITEMS>(ws, row, key);
    select_top<ITEMS>(key, (uint32_t)T, sm);
    for (int tx = threadIdx.x; tx < T; tx += kBlock)
        transform_emit(p, row, tx, candidate_pos(ws, row, sm.sel[tx] & 0x7fffffff));
}

// ------------------------------------------------------ unfused mask/map
// sglang/srt/layers/attention/v1_deepseek/kernels.py:444-472.
__global__ void mask_fine_kernel(float* scores, int64_t stride, const void* selected, int32_t sel64,
                                 const int32_t* rt, const int32_t* members, const int32_t* lens,
                                 const int32_t* takes, int32_t maxp, int32_t take_stride, int32_t width,
                                 int32_t sink_cap, int32_t window) {
    const int64_t row = blockIdx.y;
    const int32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= width) return;
    const int32_t n = lens[row];
    const int32_t take = takes[row];
    const int32_t sink = min(n, sink_cap);
    const int32_t tail = max(sink, min(max(n - 1, 0) / 1024 * 1024, max(sink, n - window)));
    const int32_t count = take * 64 + sink + n - tail;
    const bool fine = j < take * 64;
    int32_t logical = -1;
    if (fine && j / 64 < take_stride) {
        const int32_t rank = sel64 ? (int32_t) static_cast<const int64_t*>(selected)[row * take_stride + j / 64]
                                   : static_cast<const int32_t*>(selected)[row * take_stride + j / 64];
        if (rank >= 0 && rank < maxp) {
            const int32_t page = rt[row * maxp + rank];
            if (page >= 0) logical = members[(int64_t)page * 64 + (j & 63)];
        }
    }
    const bool good = j < count && (!fine || (logical >= sink && logical < tail));
    if (!good) scores[row * stride + j] = -__builtin_huge_valf();
}

// sglang/srt/layers/attention/v1_deepseek/kernels.py:323-376.
__global__ void output_ids_kernel(const int32_t* raw_in, const float* scores, int64_t stride,
                                  const int32_t* members, const int32_t* rt, const int32_t* nt,
                                  const void* selected, int32_t sel64, const int32_t* lens,
                                  const int32_t* takes, int32_t* out, int32_t* logical_out,
                                  const int32_t* ft, int32_t maxp, int32_t np, int32_t take_stride,
                                  int32_t width, int32_t topk, int32_t sink_cap, int32_t window,
                                  int32_t map_physical, int32_t direct_fine, int32_t fp) {
    const int64_t row = blockIdx.y;
    const int32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= topk) return;
    const int32_t raw = raw_in[row * topk + j];
    const int32_t take = takes[row];
    const int32_t n = lens[row];
    const int32_t sink = min(n, sink_cap);
    const int32_t tail = max(sink, min(max(n - 1, 0) / 1024 * 1024, max(sink, n - window)));
    bool valid = raw >= 0 && raw < width;
    int32_t logical = -1;
    if (valid) {
        if (raw < take * 64) {
            int32_t page = -1;
            if (direct_fine) {
                if (raw / 64 < fp) page = ft[row * fp + raw / 64];
            } else if (raw / 64 < take_stride) {
                const int32_t rank = sel64 ? (int32_t) static_cast<const int64_t*>(selected)[row * take_stride + raw / 64]
                                           : static_cast<const int32_t*>(selected)[row * take_stride + raw / 64];
                if (rank >= 0 && rank < maxp) page = rt[row * maxp + rank];
            }
            if (page >= 0) logical = members[(int64_t)page * 64 + (raw & 63)];
        } else {
            const int32_t off = raw - take * 64;
            logical = off < sink ? off : tail + off - sink;
        }
        const float sc = scores[row * stride + raw];
        valid = sc != -__builtin_huge_valf() && logical >= 0 && logical < n && logical / 64 < np;
    }
    const int64_t dst = row * topk + j;
    if (map_physical) out[dst] = valid ? nt[row * np + logical / 64] * 64 + (logical & 63) : -1;
    logical_out[dst] = valid ? logical : -1;
}

template <typename P>
int launch_single(void (*k4)(P), void (*k8)(P), void (*k16)(P), void (*k32)(P), int32_t cols, int32_t batch,
                  const P& p, hipStream_t st, const char* name) {
    auto kern = cols <= 4096 ? k4 : cols <= 8192 ? k8 : cols <= 16384 ? k16 : k32;
    hipLaunchKernelGGL(kern, dim3(batch), dim3(kBlock), 0, st, p);
    return V1_LAUNCHED(name);
}

template <typename P>
int launch_segmented(void (*seg)(P, Workspace), void (*m8)(P, Workspace), void (*m16)(P, Workspace),
                     void (*m32)(P, Workspace), int32_t cols, int32_t batch, int32_t topk, void* wsp,
                     int64_t ws_bytes, const P& p, hipStream_t st, const char* name) {
    V1_REQUIRE(wsp != nullptr && ws_bytes >= workspace_bytes(batch, cols, topk),
               "%s: rows longer than %d columns need a workspace of %lld bytes", name, kSegment,
               (long long)workspace_bytes(batch, cols, topk));
    const Workspace ws = make_workspace(wsp, batch, cols, topk);
    const int64_t cand = (int64_t)ws.nseg * topk;
    V1_REQUIRE(cand <= 32 * kBlock, "%s: %d columns exceed the %lld supported at topk %d", name, cols,
               (long long)(32 * kBlock / topk) * kSegment, topk);
    hipLaunchKernelGGL(seg, dim3(ws.nseg, batch), dim3(kBlock), 0, st, p, ws);
    int rc = V1_LAUNCHED(name);
    if (rc != V1_OK) return rc;
    auto merge = cand <= 8192 ? m8 : cand <= 16384 ? m16 : m32;
    hipLaunchKernelGGL(merge, dim3(batch), dim3(kBlock), 0, st, p, ws);
    return V1_LAUNCHED(name);
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int64_t v1_topk_workspace(int32_t batch, int32_t cols, int32_t topk) {
    if (cols <= kSegment || batch <= 0 || topk <= 0) return 0;
    return workspace_bytes(batch, cols, topk);
}

extern "C" int v1_topk(const v1_topk_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "topk: null args");
    V1_REQUIRE(a->batch >= 0 && a->cols >= 0 && a->pages > 0, "topk: bad shape");
    V1_REQUIRE(a->topk > 0 && a->topk <= V1_MAX_TOPK, "topk: topk must be in (0, 2048]");
    V1_REQUIRE(a->window >= 0 && a->window <= 4096, "topk: window must be in [0, 4096]");
    V1_REQUIRE(a->selected_bits == 32 || a->selected_bits == 64, "topk: selected must be int32 or int64");
    V1_REQUIRE(a->expansion_stride == 0 || a->expansion_stride == a->topk * 4 + 64, "topk: invalid expansion buffer");
    V1_REQUIRE(!a->direct_fine || a->fine_table_cols >= a->take_stride, "topk: invalid direct fine table");
    V1_REQUIRE(a->member_pages > 0, "topk: empty members");
    if (a->batch == 0) return V1_OK;
    V1Params p{a->scores, a->score_stride, a->cols, a->fine_lens, a->members, a->member_pages, a->rt, a->nt,
               a->pages, a->selected, a->selected_bits == 64, a->take_stride, a->lens, a->takes, a->physical,
               a->logical, a->raw, a->topk, a->window, a->mask, a->expanded, a->expansion_stride,
               a->physical_output, a->bucket_from_rank, a->fine_table, a->fine_table_cols, a->direct_fine};
    hipStream_t st = as_stream(stream);
    if (a->cols <= kSegment)
        return launch_single<V1Params>(v1_topk_rows<4>, v1_topk_rows<8>, v1_topk_rows<16>, v1_topk_rows<32>,
                                       a->cols, a->batch, p, st, "v1_topk");
    return launch_segmented<V1Params>(v1_topk_segments, v1_topk_merge<8>, v1_topk_merge<16>, v1_topk_merge<32>,
                                      a->cols, a->batch, a->topk, a->workspace, a->workspace_bytes, p, st,
                                      "v1_topk");
}

extern "C" int v1_topk_transform(const v1_topk_transform_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "topk_transform: null args");
    V1_REQUIRE(a->batch >= 0 && a->cols >= 0, "topk_transform: bad shape");
    V1_REQUIRE(a->topk > 0 && a->topk <= V1_MAX_TOPK, "topk_transform: topk must be in (0, 2048]");
    V1_REQUIRE(a->page_bits >= 0 && a->page_bits < 31, "topk_transform: bad page_bits");
    if (a->batch == 0) return V1_OK;
    TransformParams p{a->scores, a->score_stride, a->cols, a->seq_lens, a->page_table, a->page_table_stride,
                      a->page_table_cols, a->page_bits, a->page_indices, a->raw_indices, a->topk};
    hipStream_t st = as_stream(stream);
    if (a->cols <= kSegment)
        return launch_single<TransformParams>(transform_rows<4>, transform_rows<8>, transform_rows<16>,
                                              transform_rows<32>, a->cols, a->batch, p, st, "topk_transform");
    return launch_segmented<TransformParams>(transform_segments, transform_merge<8>, transform_merge<16>,
                                             transform_merge<32>, a->cols, a->batch, a->topk, a->workspace,
                                             a->workspace_bytes, p, st, "topk_transform");
}

extern "C" int v1_mask_fine(float* scores, int64_t score_stride, const void* selected, int32_t selected_bits,
                            const int32_t* rt, const int32_t* members, const int32_t* lens, const int32_t* takes,
                            int32_t rows, int32_t maxp, int32_t take_stride, int32_t width, int32_t sink,
                            int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && width >= 0 && maxp > 0, "mask_fine: bad shape");
    V1_REQUIRE(selected_bits == 32 || selected_bits == 64, "mask_fine: selected must be int32 or int64");
    if (rows == 0 || width == 0) return V1_OK;
    hipLaunchKernelGGL(mask_fine_kernel, dim3((uint32_t)cdiv(width, 256), rows), dim3(256), 0, as_stream(stream),
                       scores, score_stride, selected, selected_bits == 64, rt, members, lens, takes, maxp,
                       take_stride, width, sink, window);
    return V1_LAUNCHED("mask_fine");
}

extern "C" int v1_output_ids(const int32_t* raw, const float* scores, int64_t score_stride, const int32_t* members,
                             const int32_t* rt, const int32_t* nt, const void* selected, int32_t selected_bits,
                             const int32_t* lens, const int32_t* takes, int32_t* out, int32_t* logical,
                             const int32_t* ft, int32_t rows, int32_t maxp, int32_t np, int32_t take_stride,
                             int32_t width, int32_t topk, int32_t sink, int32_t window, int32_t map_physical,
                             int32_t direct_fine, int32_t fp, void* stream) {
    V1_REQUIRE(rows >= 0 && topk >= 0 && maxp > 0 && np > 0, "output_ids: bad shape");
    V1_REQUIRE(selected_bits == 32 || selected_bits == 64, "output_ids: selected must be int32 or int64");
    if (rows == 0 || topk == 0) return V1_OK;
    hipLaunchKernelGGL(output_ids_kernel, dim3((uint32_t)cdiv(topk, 256), rows), dim3(256), 0, as_stream(stream),
                       raw, scores, score_stride, members, rt, nt, selected, selected_bits == 64, lens, takes, out,
                       logical, ft, maxp, np, take_stride, width, topk, sink, window, map_physical, direct_fine, fp);
    return V1_LAUNCHED("output_ids");
}
