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
// Design: one 512-thread work-group selects over up to 40960 positions with
// under 40 KiB of LDS, so four work-groups (rows) share a CU and the HBM
// streams of some rows overlap the LDS selection of others.
//  1. 2048 keys sampled in 64 runs of 32 (one 128-byte line each: 8 KB of a
//     row's lines) give a pivot that about 1.2*T of the row's keys exceed.
//  2. One streaming pass, wave-independent (no barriers), sends every score at
//     or above the pivot to an LDS candidate buffer (a float compare per score,
//     ballot-counted slots per wave).
//  3. LDS radix passes over the candidates (the first digit starts where the
//     largest and smallest candidate differ) give the T-th largest key tau and
//     the number r of tau-valued keys to take.
//  4. Position bitmaps of "> tau" and "== tau" plus a block prefix of their
//     popcounts give each winner its output slot: (> tau before it) +
//     min(== tau before it, r).  No sort is needed and the order is exact;
//     each winner is written straight to its output slot.
// When the pivot misses (fewer than T or more than kCandMax keys at or above
// it) a second pivot, aimed by the observed count, is streamed once more; a
// second miss runs the same steps exactly on the whole row (statistics, radix
// passes), streamed again.
// Rows longer than 40960 columns (32768 in batches of fewer than 512 rows,
// where more, shorter segments keep more of the GPU busy) are cut into
// segments whose Top-T land in a workspace; a merge work-group selects from
// their union.
#include <algorithm>
#include <cstddef>

#include "common.h"

namespace v1 {
namespace {

constexpr int kBlock = 512;
constexpr int kWaves = kBlock / kWave;  // 8
constexpr int kSpan = 40960;            // positions one work-group selects over
constexpr int kWords = kSpan / 32;      // position bitmap words
constexpr int kDigitBits = 10;          // radix digit width
constexpr int kHist = 1 << kDigitBits;  // histogram bins, 2 per thread
constexpr int kHistWords = kHist > kWords ? kHist : kWords;  // histograms; bitmap word prefixes
constexpr int kCandMax = 3584;
constexpr int kCandPerThread = kCandMax / kBlock;  // 7
constexpr int kSampleRuns = 64;                    // pivot sample: runs of 32 keys (128 bytes)
constexpr int kTableBits = 6;                      // page size (log2) from which a row's table fits kBlock ints
constexpr uint32_t kNegInfKey = 0x007fffffu;
constexpr uint32_t kPosInfKey = 0xff800000u;  // key of +inf; keys above it are positive NaNs
constexpr uint32_t kNegInfBits = 0xff800000u;  // float bits of -inf
// Word 3 of a raw buffer descriptor (stride 0, 32-bit dwords): loads at byte
// offsets at or past the descriptor's length return zeros.
constexpr int32_t kRawDword = 0x00020000;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
static_assert(kHist % kBlock == 0 && kWords % 256 == 0 && kCandMax % kBlock == 0, "work split");
static_assert(kSampleRuns * 32 == 4 * kBlock, "eight threads per sample run");

struct alignas(16) SelSmem {  // (arrays at 16-byte offsets: read as 16-byte words)
    uint32_t hist[kHistWords];  // radix histograms; bitmap word prefixes
    uint32_t cand_key[kCandMax];  // (after the ranks of a transform row: its selected positions in slot order)
    uint16_t cand_pos[kCandMax];
    uint32_t gt_bits[kWords];  // positions with key > tau
    uint32_t eq_bits[kWords];  // positions with key == tau
    uint32_t red[4 * kWaves];
    uint32_t bc[4];
    uint32_t ncand;
    int32_t maskpage[kSpan / 64];  // V1 mask: page per selected rank, -1 when unmasked; or a row's page table
};
static_assert(sizeof(SelSmem) <= 40 * 1024, "four work-groups per CU");
static_assert(alignof(SelSmem) >= 16, "16-byte LDS words at any placement of the struct");
static_assert(offsetof(SelSmem, gt_bits) % 16 == 0 && offsetof(SelSmem, eq_bits) % 16 == 0, "16-byte words");
static_assert(offsetof(SelSmem, cand_key) % 8 == 0 && kCandMax * 4 >= 2 * 2048, "T <= 2048 staged positions");

__device__ __forceinline__ uint32_t readlane(uint32_t v, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

// Wave-wide max (kOp 0), min (1) or sum (2) on DPP lane moves: row_shr
// 1/2/4/8 inside each 16-lane row, then row_bcast 15 / 31 across rows, which
// leaves the result in lane 63.
template <int kOp>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
    constexpr int kId = kOp == 1 ? -1 : 0;
    auto f = [](uint32_t a, uint32_t b) { return kOp == 0 ? max(a, b) : kOp == 1 ? min(a, b) : a + b; };
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = f(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, kWave - 1);
}

// Block-wide max / min / count; every thread gets the result.  sm.red is read
// after the one barrier: the caller passes another barrier before sm.red is
// written again.
__device__ __forceinline__ void block_stats(uint32_t& mx, uint32_t& mn, uint32_t& n, SelSmem& sm) {
    mx = wave_reduce<0>(mx);
    mn = wave_reduce<1>(mn);
    n = wave_reduce<2>(n);
    const int w = threadIdx.x / kWave;
    if (__lane_id() == 0) {
        sm.red[w] = mx;
        sm.red[kWaves + w] = mn;
        sm.red[2 * kWaves + w] = n;
    }
    __syncthreads();
    mx = 0u;
    mn = 0xffffffffu;
    n = 0u;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
        mx = max(mx, sm.red[k]);
        mn = min(mn, sm.red[kWaves + k]);
        n += sm.red[2 * kWaves + k];
    }
    // (uniform: kept in scalar registers)
    mx = __builtin_amdgcn_readfirstlane(mx);
    mn = __builtin_amdgcn_readfirstlane(mn);
    n = __builtin_amdgcn_readfirstlane(n);
}

__device__ __forceinline__ void key_stats(uint32_t k, uint32_t& mx, uint32_t& mn, uint32_t& n) {
    const bool real = k > kNegInfKey;
    mx = real ? max(mx, k) : mx;
    mn = real ? min(mn, k) : mn;
    n += real ? 1u : 0u;
}

// Descending scan of hist[0..kHist): the bin holding the `rank`-th largest
// counted key (1 <= rank <= the count), the count above it and the bin's own
// count.  Wave 0 scans alone: lane l sums the 32 bins below kHist - 32 l
// (eight 16-byte reads), a lane prefix finds the owning lane, and its 32 bins,
// one per lane, a second prefix finds the bin.  Every bin read is zeroed, so
// the histogram is clear for the next pass without a clearing step.  Call
// after the barrier that completes the histogram; ends with a barrier.
__device__ __forceinline__ void find_bin(uint32_t rank, SelSmem& sm, uint32_t& bin, uint32_t& above,
                                         uint32_t& inbin) {
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        constexpr int kPer = kHist / kWave;  // bins per lane
        uint4* h4 = reinterpret_cast<uint4*>(sm.hist + kHist - kPer * (lane + 1));
        uint32_t local = 0;
#pragma unroll
        for (int i = 0; i < kPer / 4; ++i) {
            const uint4 v = h4[i];
            local += v.x + v.y + v.z + v.w;
        }
        const uint32_t incl = wave_inclusive_sum(local);
        const uint64_t own = __builtin_amdgcn_ballot_w64(incl >= rank);
        if (own != 0) {
            const int L = (int)__builtin_ctzll(own);
            const uint32_t excl = readlane(incl - local, L);
            const uint32_t top = (uint32_t)(kHist - 1 - kPer * L);
            const uint32_t c = lane < kPer ? sm.hist[top - lane] : 0u;
            const uint32_t ci = wave_inclusive_sum(c);
            const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < kPer && excl + ci >= rank);
            if (lane == (int)__builtin_ctzll(hit)) {
                sm.bc[0] = top - lane;
                sm.bc[1] = excl + ci - c;
                sm.bc[2] = c;
            }
        }
        // (after the reads above: one wave's LDS accesses complete in order)
#pragma unroll
        for (int i = 0; i < kPer / 4; ++i) h4[i] = make_uint4(0u, 0u, 0u, 0u);
        if (threadIdx.x == 0) sm.bc[3] = 0;  // append counter of small_bin_select
    }
    __syncthreads();
    bin = __builtin_amdgcn_readfirstlane(sm.bc[0]);
    above = __builtin_amdgcn_readfirstlane(sm.bc[1]);
    inbin = __builtin_amdgcn_readfirstlane(sm.bc[2]);
}

__device__ __forceinline__ void clear_hist(SelSmem& sm) {
#pragma unroll
    for (int i = 0; i < kHist / kBlock; ++i) sm.hist[threadIdx.x + i * kBlock] = 0;
}

// Digit window of a pass: bits [shift, shift+bits) under the fixed prefix.
struct Radix {
    uint32_t prefix, pmask, remaining;
    int shift;  // bits still unresolved below the prefix
    __device__ __forceinline__ void start(uint32_t mx, uint32_t mn, uint32_t T) {
        const int hb = 31 - __builtin_clz(mx ^ mn);
        pmask = hb == 31 ? 0u : ~((2u << hb) - 1u);
        prefix = mx & pmask;
        remaining = T;
        shift = hb + 1;
    }
    __device__ __forceinline__ int bits() const { return shift < kDigitBits ? shift : kDigitBits; }
    __device__ __forceinline__ bool counts(uint32_t k, bool real_only) const {
        return (k & pmask) == prefix && (!real_only || k > kNegInfKey);
    }
    __device__ __forceinline__ uint32_t digit(uint32_t k) const {
        return (k >> (shift - bits())) & ((1u << bits()) - 1u);
    }
    // after the histogram of this pass is in sm.hist (and a barrier); returns
    // the count of the bin now fixed in the prefix
    __device__ __forceinline__ uint32_t finish(SelSmem& sm) {
        uint32_t bin, above, inbin;
        find_bin(remaining, sm, bin, above, inbin);
        const int b = bits();
        shift -= b;
        remaining -= above;
        prefix |= bin << shift;
        pmask |= ((1u << b) - 1u) << shift;
        return inbin;
    }
};

// Position ranks of the winners: builds the "> tau" / "== tau" bitmaps from
// `mark(emit)` and the block prefix of their packed popcounts; `place(emit)`
// then visits each marked item again and writes it to its slot.
struct Ranker {
    __device__ __forceinline__ static void clear(SelSmem& sm) {
        for (int i = threadIdx.x; i < kWords; i += kBlock) {
            sm.gt_bits[i] = 0;
            sm.eq_bits[i] = 0;
        }
    }
    __device__ __forceinline__ static void mark(SelSmem& sm, uint32_t pos, bool gt, bool eq) {
        if (gt) atomicOr(&sm.gt_bits[pos >> 5], 1u << (pos & 31));
        if (eq) atomicOr(&sm.eq_bits[pos >> 5], 1u << (pos & 31));
    }
    // word prefixes: hist[w] = packed (gt | eq << 16) count before word w;
    // wave 0 scans the kWords words, kWords / 64 per lane
    __device__ __forceinline__ static void scan(SelSmem& sm) {
        if (threadIdx.x < kWave) {
            const int lane = threadIdx.x;
            constexpr int kWpl = kWords / kWave;  // words per lane
            static_assert(kWpl % 4 == 0, "16-byte LDS words");
            // (16-byte LDS accesses: words kWpl lane .. kWpl lane + kWpl - 1)
            const uint4* g4 = reinterpret_cast<const uint4*>(sm.gt_bits + kWpl * lane);
            const uint4* e4 = reinterpret_cast<const uint4*>(sm.eq_bits + kWpl * lane);
            uint32_t c[kWpl];
            uint32_t local = 0;
#pragma unroll
            for (int q = 0; q < kWpl / 4; ++q) {
                const uint4 g = g4[q], e = e4[q];
                c[4 * q + 0] = (uint32_t)__popc(g.x) | ((uint32_t)__popc(e.x) << 16);
                c[4 * q + 1] = (uint32_t)__popc(g.y) | ((uint32_t)__popc(e.y) << 16);
                c[4 * q + 2] = (uint32_t)__popc(g.z) | ((uint32_t)__popc(e.z) << 16);
                c[4 * q + 3] = (uint32_t)__popc(g.w) | ((uint32_t)__popc(e.w) << 16);
                local += c[4 * q] + c[4 * q + 1] + c[4 * q + 2] + c[4 * q + 3];
            }
            uint32_t run = wave_inclusive_sum(local) - local;
            uint4* h4 = reinterpret_cast<uint4*>(sm.hist + kWpl * lane);
#pragma unroll
            for (int q = 0; q < kWpl / 4; ++q) {
                uint4 o;
                o.x = run;
                run += c[4 * q];
                o.y = run;
                run += c[4 * q + 1];
                o.z = run;
                run += c[4 * q + 2];
                o.w = run;
                run += c[4 * q + 3];
                h4[q] = o;
            }
        }
        __syncthreads();
    }
    // output slot of a marked position, or -1 for an eq item past the first r
    __device__ __forceinline__ static int32_t slot(const SelSmem& sm, uint32_t pos, bool gt, uint32_t r) {
        const uint32_t w = pos >> 5, below = (1u << (pos & 31)) - 1u;
        const uint32_t pre = sm.hist[w];
        const uint32_t g = (pre & 0xffffu) + (uint32_t)__popc(sm.gt_bits[w] & below);
        const uint32_t e = (pre >> 16) + (uint32_t)__popc(sm.eq_bits[w] & below);
        if (gt) return (int32_t)(g + min(e, r));
        return e < r ? (int32_t)(g + e) : -1;
    }
};

// Pivot from the sampled keys sk (threads 8r..8r+7 hold run r of 32 keys;
// block statistics smax / smin / scnt) such that about target * T of the n
// keys are expected at or above it.  With a histogram (scnt > 0 and
// smax != smin) it ends with find_bin's barrier; otherwise it passes no
// barrier.  Either way it leaves sm.hist clear, and it writes no LDS word on
// the no-histogram branch, so the caller may append candidates (sm.cand_*,
// sm.ncand) at once but must pass a barrier before writing sm.red or sm.bc.
__device__ uint32_t choose_pivot(const uint32_t (&sk)[4], uint32_t smax, uint32_t smin, uint32_t scnt, int32_t n,
                                 uint32_t T, float target, SelSmem& sm) {
    uint32_t pivot = kNegInfKey + 1;
    if (scnt > 0 && smax == smin) {
        pivot = smin;
    } else if (scnt > 0) {
        Radix rx;
        rx.start(smax, smin, 1);
        const int lo = rx.shift > kDigitBits ? rx.shift - kDigitBits : 0;
        // (the empty asm keeps the bin addresses from being computed once
        // before the caller's attempt loop and held, spilled, across the stream)
        uint32_t k[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            k[e] = sk[e];
            asm volatile("" : "+v"(k[e]));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (k[e] > kNegInfKey) atomicAdd(&sm.hist[(k[e] >> lo) & (kHist - 1u)], 1u);
        __syncthreads();
        const uint32_t want = (uint32_t)min((float)scnt, (float)scnt * (float)T * target / (float)n + 16.f);
        uint32_t bin, above, inbin;
        find_bin(want, sm, bin, above, inbin);
        // Expected candidates with the pivot at the bin's lower edge (every
        // sample of the bin passes) or just above the bin (none passes).
        // (floor(a * n / scnt) <= K  <=>  a * n < (K + 1) * scnt, and
        // floor(a * n / scnt) >= K  <=>  a * n >= K * scnt: no divisions)
        const uint64_t lo_n = (uint64_t)(above + inbin) * (uint64_t)n, hi_n = (uint64_t)above * (uint64_t)n;
        if (lo_n < ((uint64_t)kCandMax * 7 / 8 + 1) * scnt || lo == 0) {
            pivot = rx.prefix | (bin << lo);
        } else if (hi_n >= ((uint64_t)T * 9 / 8) * scnt && bin + 1 < (uint32_t)kHist) {
            pivot = rx.prefix | ((bin + 1) << lo);
        } else {
            // refine inside the bin on the next digit
            const int lo2 = lo > kDigitBits ? lo - kDigitBits : 0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (k[e] > kNegInfKey && ((k[e] >> lo) & (kHist - 1u)) == bin && (k[e] & rx.pmask) == rx.prefix)
                    atomicAdd(&sm.hist[(k[e] >> lo2) & ((1u << (lo - lo2)) - 1u)], 1u);
            __syncthreads();
            uint32_t bin2, above2, inbin2;
            find_bin(want - above, sm, bin2, above2, inbin2);
            pivot = rx.prefix | (bin << lo) | (bin2 << lo2);
        }
        pivot = max(pivot, kNegInfKey + 1);
    }
    return pivot;
}

// The candidate test and LDS append for one wave's kBatch loads of 4 entries
// (load u at step s0 + u * kWaves, lane's entries p..p+3).  With a pivot
// above +0 (int_test) the key test is one signed compare of the raw bits
// against the pivot's float bits: negative scores and -NaNs are negative as
// int32, +0 / -0 lie below the pivot, and +inf / +NaNs order above every
// finite score, as their keys do.
template <class Src, int kBatch>
__device__ __forceinline__ void take_candidates(const uint32_t (&v)[kBatch][4], int32_t s0, uint32_t pivot,
                                                bool float_test, float fpivot, bool int_test, SelSmem& sm) {
    const int lane = __lane_id();
    // slots are allocated per pair of batches (keeps the lane masks in
    // scalar registers)
#pragma unroll
    for (int h = 0; h < kBatch; h += 2) {
        bool c[2][4];
        if (Src::kFloats && int_test) {
            const int32_t ipivot = (int32_t)__float_as_uint(fpivot);
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) c[u][e] = (int32_t)v[h + u][e] >= ipivot;
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bool nan = false;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = __uint_as_float(v[h + u][e]);
                    c[u][e] = Src::kFloats ? x >= fpivot : v[h + u][e] >= pivot;
                    nan |= x != x;
                }
                if (Src::kFloats && (!float_test || __builtin_amdgcn_ballot_w64(nan) != 0)) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) c[u][e] = score_key(__uint_as_float(v[h + u][e])) >= pivot;
                }
            }
        }
        uint64_t m[2][4];
        uint32_t pre[2][4], total = 0;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                m[u][e] = __builtin_amdgcn_ballot_w64(c[u][e]);
                pre[u][e] = total;
                total += (uint32_t)__builtin_popcountll(m[u][e]);
            }
        if (total == 0) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sm.ncand, total);
        base = readlane(base, 0);
        // A pair that would pass kCandMax writes nothing: ncand then ends
        // above kCandMax, and the attempt's buffer is not used.
        if (base + total > (uint32_t)kCandMax) continue;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int32_t p = (s0 + (h + u) * kWaves) * 256 + 4 * lane;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (c[u][e]) {
                    // slot base + pre + (lanes below with the entry): scalar
                    // row pointers plus one shifted add per array
                    const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m[u][e] >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m[u][e], 0u));
                    (sm.cand_key + base + pre[u][e])[below] = v[h + u][e];
                    (sm.cand_pos + base + pre[u][e])[below] = (uint16_t)(p + e);
                }
            }
        }
    }
}

// Step 2: every entry at or above the pivot goes to the LDS candidate buffer
// (sm.ncand counts them all; the first kCandMax are kept).  Score rows are
// tested as floats against the pivot's float (key order and float order
// agree on every non-NaN score, with -0 == +0) and stored as raw bits, which
// the selection turns into keys; a wave batch holding a NaN, or a pivot in
// the NaN key range, takes the exact key test.  Slots come from one LDS
// allocation per wave and pair of batches (ballot counts, mbcnt ranks).
// Sources with a buffer descriptor (Src::kBuffer) keep a ring of loads in
// flight per wave while they test; others load kBatch, then test.
template <class Src>
__device__ __forceinline__ void stream_candidates(const Src& src, uint32_t pivot, SelSmem& sm) {
    // (the wave index as a scalar: the loop below branches per wave)
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = __lane_id();
    const int32_t n = src.n;
    const int32_t steps = (n + 255) / 256;
    constexpr int kBatch = 4;
    constexpr int32_t kStride = kWaves * kBatch;  // steps per wave iteration
    const bool float_test = Src::kFloats && pivot <= kPosInfKey;
    const bool int_test = Src::kFloats && pivot > 0x80000000u;  // pivot score above +0
    const float fpivot = key_score(pivot);
    if constexpr (Src::kBuffer) {
        // A ring of kRing 1 KB loads per wave over the wave's (at most
        // kMaxLoads) loads, fully unrolled: the loads of a pair of slots are
        // waited for, tested, and the slots reloaded kRing loads ahead, so up
        // to kRing - 2 loads stay in flight while a pair is tested.  Every
        // load is issued (past the row's end the buffer descriptor returns
        // zeros without a memory access), which keeps the wait counts exact.
        constexpr int kRing = 8;
        constexpr int kMaxLoads = kSpan / (256 * kWaves);  // 16: n <= kSpan
        const auto rs = src.rsrc();
        const int32_t nload = (steps - w + kWaves - 1) / kWaves;  // this wave's loads: steps w + i * kWaves
        uint32_t r[kRing][4];
        auto issue = [&](uint32_t (&x)[4], int i) {
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * ((w + i * kWaves) * 256 + 4 * lane), 0, 0);
            x[0] = q[0];
            x[1] = q[1];
            x[2] = q[2];
            x[3] = q[3];
        };
        // (in slot order: the scheduler would otherwise reorder the loads,
        // and the first wait would then cover the whole ring)
#pragma unroll
        for (int j = 0; j < kRing; ++j) {
            issue(r[j], j);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < kMaxLoads; i += 2) {
            uint32_t(&x)[2][4] = *reinterpret_cast<uint32_t(*)[2][4]>(&r[i % kRing]);
            if (i < nload) {
                const int32_t s0 = w + i * kWaves;
                // entries past n read as zeros: the pair holding the row's end sets them to -inf
                if ((s0 + kWaves + 1) * 256 > n) {
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if ((s0 + u * kWaves) * 256 + 4 * lane + e >= n) x[u][e] = kNegInfBits;
                }
                take_candidates<Src, 2>(x, s0, pivot, float_test, fpivot, int_test, sm);
            }
            if (i + kRing < kMaxLoads) {
                issue(x[0], i + kRing);
                issue(x[1], i + 1 + kRing);
            }
        }
    } else {
        for (int32_t s0 = w; s0 < steps; s0 += kStride) {
            uint32_t v[kBatch][4];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) src.load_raw4((s0 + u * kWaves) * 256 + 4 * lane, v[u]);
            take_candidates<Src, kBatch>(v, s0, pivot, float_test, fpivot, int_test, sm);
        }
    }
}

// The radix select's end when the bin just fixed in rx's prefix holds at most
// one wave of keys: they are appended to sm.hist[0..inbin) (the histogram is
// clear between passes), and wave 0 ranks them against each other, which
// resolves every remaining bit at once.  tau is the rx.remaining-th largest
// key of the bin and r the number of keys equal to tau that are taken (the
// radix select's final prefix and remaining).  The list is cleared again.
template <int kN>
__device__ __forceinline__ void small_bin_select(const uint32_t (&ck)[kN], const Radix& rx, uint32_t inbin,
                                                 SelSmem& sm, uint32_t& tau, uint32_t& r) {
    // one LDS allocation per wave (ballot counts, mbcnt ranks)
    const int lane = __lane_id();
    uint64_t bal[kN];
    uint32_t pre[kN], total = 0;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
        bal[i] = __builtin_amdgcn_ballot_w64(rx.counts(ck[i], true));
        pre[i] = total;
        total += (uint32_t)__builtin_popcountll(bal[i]);
    }
    if (total > 0) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sm.bc[3], total);
        base = readlane(base, 0);
#pragma unroll
        for (int i = 0; i < kN; ++i)
            if (rx.counts(ck[i], true))
                sm.hist[base + pre[i] +
                        __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[i] >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)bal[i], 0u))] = ck[i];
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
        // every lane reads the list as 16-byte words (bins past it are zero,
        // below every real key)
        const uint32_t k = lane < (int)inbin ? sm.hist[lane] : 0u;
        uint32_t gt = 0, eq = 0;
        for (uint32_t j = 0; j < inbin; j += 4) {
            const uint4 q = *reinterpret_cast<const uint4*>(sm.hist + j);
            gt += (q.x > k ? 1u : 0u) + (q.y > k ? 1u : 0u) + (q.z > k ? 1u : 0u) + (q.w > k ? 1u : 0u);
            eq += (q.x == k ? 1u : 0u) + (q.y == k ? 1u : 0u) + (q.z == k ? 1u : 0u) + (q.w == k ? 1u : 0u);
        }
        const uint64_t hit =
            __builtin_amdgcn_ballot_w64(lane < (int)inbin && gt < rx.remaining && rx.remaining <= gt + eq);
        if (lane == (int)__builtin_ctzll(hit)) {
            sm.bc[0] = k;
            sm.bc[1] = rx.remaining - gt;
        }
        if (lane < (int)inbin) sm.hist[lane] = 0;  // after the reads above (in-order LDS)
    }
    __syncthreads();
    tau = __builtin_amdgcn_readfirstlane(sm.bc[0]);
    r = __builtin_amdgcn_readfirstlane(sm.bc[1]);
}

// Step 3: the T-th largest key tau of the keys held in ck[] across the
// work-group (block statistics cmax / cmin of the real keys, at least T of
// them), and r, the number of keys equal to tau that are taken.
template <int kN>
__device__ __forceinline__ void radix_tau(const uint32_t (&ck)[kN], uint32_t cmax, uint32_t cmin, uint32_t T,
                                          SelSmem& sm, uint32_t& tau, uint32_t& r) {
    tau = cmax;
    r = T;
    if (cmax == cmin) return;
    Radix rx;
    rx.start(cmax, cmin, T);
    while (rx.shift > 0) {
#pragma unroll
        for (int i = 0; i < kN; ++i)
            if (rx.counts(ck[i], true)) atomicAdd(&sm.hist[rx.digit(ck[i])], 1u);
        __syncthreads();
        const uint32_t inbin = rx.finish(sm);
        if (rx.shift > 0 && inbin <= (uint32_t)kWave) {
            small_bin_select(ck, rx, inbin, sm, tau, r);
            return;
        }
    }
    tau = rx.prefix;
    r = rx.remaining;
}

// Steps 3 and 4 over ncand (T <= ncand <= kCandMax) buffered candidates.
// Ends with a barrier.
template <class Src, class Emit>
__device__ void select_candidates(uint32_t ncand, uint32_t T, SelSmem& sm, const Emit& emit) {
    const int t = threadIdx.x;
    // 3. radix select on the candidates (kCandPerThread per thread, slot q = i*kBlock + t)
    uint32_t ck[kCandPerThread];
    uint32_t cmax = 0, cmin = 0xffffffffu, cc = 0;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {
        const uint32_t q = i * kBlock + t;
        ck[i] = q < ncand ? (Src::kFloats ? score_key(__uint_as_float(sm.cand_key[q])) : sm.cand_key[q]) : 0u;
        key_stats(ck[i], cmax, cmin, cc);
    }
    block_stats(cmax, cmin, cc, sm);
    uint32_t tau, r;
    radix_tau(ck, cmax, cmin, T, sm, tau, r);
    // 4. position ranks
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {
        const uint32_t q = i * kBlock + t;
        if (q < ncand) Ranker::mark(sm, sm.cand_pos[q], ck[i] > tau, ck[i] == tau);
    }
    __syncthreads();
    Ranker::scan(sm);
    int32_t at[kCandPerThread];
    uint32_t cp[kCandPerThread];
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {
        const uint32_t q = i * kBlock + t;
        cp[i] = q < ncand ? (uint32_t)sm.cand_pos[q] : 0u;
        at[i] = (q < ncand && ck[i] >= tau) ? Ranker::slot(sm, cp[i], ck[i] > tau, r) : -1;
    }
    emit(at, cp, ck);
    __syncthreads();
}

// Selects the T largest keys of positions [0, n) of `src` (n > T, n <= kSpan;
// ties toward the lower position).  emit(slot[], position[], key[]) takes a
// thread's batch of items (arrays of one length; slot -1 = not selected):
// every slot in [0, T) is delivered exactly once, the slots ascending by
// position.  Batches let the emitter issue all of a thread's output loads
// before its stores.  src.load4(p, k) returns the keys of positions p..p+3
// (p % 4 == 0), key 0 past n; src.load_raw4 the raw entries (float bits, -inf
// past n, when Src::kFloats; else keys).  Ends with a barrier.
template <class Src, class Emit>
__device__ void select_exact(const Src& src, uint32_t T, SelSmem& sm, const Emit& emit);

// Step 1's sample: thread t reads keys p..p+3 of run t / 8 of 32 keys, one
// 128-byte line of the row (a line-sized run costs no more fetch than a
// shorter one, and the stream re-reads the row anyway); 2048 keys in all.
__device__ __forceinline__ int32_t sample_pos(int32_t n) {
    const int t = threadIdx.x;
    return (int32_t)((((int64_t)(t >> 3) * n / kSampleRuns) & ~31ll) + 4 * (t & 7));
}

template <class Src, class Emit>
__device__ void select_sampled(const Src& src, const uint32_t (&sk)[4], uint32_t T, SelSmem& sm, const Emit& emit);

template <class Src, class Emit>
__device__ void select_stream(const Src& src, uint32_t T, SelSmem& sm, const Emit& emit) {
    uint32_t sk[4];
    src.load4(sample_pos(src.n), sk);
    select_sampled(src, sk, T, sm, emit);
}

// select_stream with the pivot sample (the keys at sample_pos) given.
template <class Src, class Emit>
__device__ void select_sampled(const Src& src, const uint32_t (&sk)[4], uint32_t T, SelSmem& sm, const Emit& emit) {
    const int t = threadIdx.x;
    const int32_t n = src.n;
    // LDS state of a selection: the histogram and the rank bitmaps start
    // clear (the first barrier below orders these stores before any use)
    clear_hist(sm);
    Ranker::clear(sm);
    if (t == 0) sm.ncand = 0;
    // 1. pivot from the sample
    uint32_t smax = 0, smin = 0xffffffffu, scnt = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) key_stats(sk[e], smax, smin, scnt);
    block_stats(smax, smin, scnt, sm);
    // Pivot attempts: the first aims at 1.2 T candidates; after a miss the
    // target is corrected by the observed candidate count and the row is
    // streamed once more; a second miss takes the exact passes below.
    float target = 1.2f;
    for (int attempt = 0; attempt < 2; ++attempt) {
        const uint32_t pivot = choose_pivot(sk, smax, smin, scnt, n, T, target, sm);
        stream_candidates(src, pivot, sm);
        __syncthreads();
        const uint32_t ncand = __builtin_amdgcn_readfirstlane(sm.ncand);
        if (ncand >= T && ncand <= (uint32_t)kCandMax) {
            select_candidates<Src>(ncand, T, sm, emit);
            return;
        }
        if (scnt == 0 || smax == smin) break;
        target *= ncand < T ? fmaxf(1.25f, 1.15f * (float)T / fmaxf((float)ncand, 1.f))
                            : fminf(0.8f, 0.9f * (float)kCandMax / (float)ncand);
        __syncthreads();  // every thread has read sm.ncand
        if (t == 0) sm.ncand = 0;
        __syncthreads();
    }
    select_exact(src, T, sm, emit);
}

// The exact steps on the whole row (the fallback after two pivot misses):
// the row's key statistics, radix passes over the row, marks and emit, each
// streaming the row again.  Ends with a barrier.
template <class Src, class Emit>
__device__ void select_exact(const Src& src, uint32_t T, SelSmem& sm, const Emit& emit) {
    const int w = threadIdx.x / kWave, lane = __lane_id();
    const int32_t n = src.n;
    const int32_t steps = (n + 255) / 256;
    uint32_t rmax = 0, rmin = 0xffffffffu, rcnt = 0;
    for (int32_t s = w; s < steps; s += kWaves) {
        uint32_t k[4];
        src.load4(s * 256 + 4 * lane, k);
#pragma unroll
        for (int e = 0; e < 4; ++e) key_stats(k[e], rmax, rmin, rcnt);
    }
    block_stats(rmax, rmin, rcnt, sm);
    uint32_t tau, r;
    if (rcnt >= T) {
        if (rmax == rmin) {
            tau = rmax;
            r = T;
        } else {
            Radix rx;
            rx.start(rmax, rmin, T);
            while (rx.shift > 0) {
                clear_hist(sm);
                __syncthreads();
                for (int32_t s = w; s < steps; s += kWaves) {
                    uint32_t k[4];
                    src.load4(s * 256 + 4 * lane, k);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (rx.counts(k[e], true)) atomicAdd(&sm.hist[rx.digit(k[e])], 1u);
                }
                __syncthreads();
                rx.finish(sm);
            }
            tau = rx.prefix;
            r = rx.remaining;
        }
    } else {
        // fewer than T keys above -inf: every key counts (-inf, NaN, padding)
        Radix rx;
        rx.prefix = 0;
        rx.pmask = 0;
        rx.remaining = T;
        rx.shift = 32;
        while (rx.shift > 0) {
            clear_hist(sm);
            __syncthreads();
            for (int32_t s = w; s < steps; s += kWaves) {
                uint32_t k[4];
                src.load4(s * 256 + 4 * lane, k);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (s * 256 + 4 * lane + e < n && rx.counts(k[e], false)) atomicAdd(&sm.hist[rx.digit(k[e])], 1u);
            }
            __syncthreads();
            rx.finish(sm);
        }
        tau = rx.prefix;
        r = rx.remaining;
    }
    for (int32_t s = w; s < steps; s += kWaves) {
        const int32_t p = s * 256 + 4 * lane;
        uint32_t k[4];
        src.load4(p, k);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (p + e < n) Ranker::mark(sm, p + e, k[e] > tau, k[e] == tau);
    }
    __syncthreads();
    Ranker::scan(sm);
    for (int32_t s = w; s < steps; s += kWaves) {
        const int32_t p = s * 256 + 4 * lane;
        uint32_t k[4], pp[4];
        int32_t at[4];
        src.load4(p, k);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            pp[e] = (uint32_t)(p + e);
            at[e] = (p + e < n && k[e] >= tau) ? Ranker::slot(sm, p + e, k[e] > tau, r) : -1;
        }
        emit(at, pp, k);
    }
    __syncthreads();
}

// Rows of at most kShort columns: the whole row is loaded into registers at
// once (kShortPer keys per thread, position 4 * (g * kBlock + t) + e for load
// g), so no sample, pivot or candidate stream is needed: the radix passes run
// over the registers, then the ranks.  Rows with fewer than T keys above -inf
// run the exact steps' all-key radix over the registers too.  Ends with a
// barrier.
constexpr int kShort = 8192;
constexpr int kShortPer = kShort / kBlock;  // 16
static_assert(kShortPer % 4 == 0, "whole 16-byte loads per thread");

template <class Src, class Emit>
__device__ void select_short(const Src& src, uint32_t T, SelSmem& sm, const Emit& emit) {
    const int t = threadIdx.x;
    const int32_t n = src.n;
    clear_hist(sm);  // (the barrier of block_stats orders these before any use)
    Ranker::clear(sm);
    uint32_t ck[kShortPer];
#pragma unroll
    for (int g = 0; g < kShortPer / 4; ++g) {
        uint32_t v[4];
        src.load_raw4(g * 4 * kBlock + 4 * t, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) ck[4 * g + e] = Src::kFloats ? score_key(__uint_as_float(v[e])) : v[e];
    }
    uint32_t cmax = 0, cmin = 0xffffffffu, cc = 0;
#pragma unroll
    for (int i = 0; i < kShortPer; ++i) key_stats(ck[i], cmax, cmin, cc);
    block_stats(cmax, cmin, cc, sm);
    auto pos = [&](int i) { return (uint32_t)(4 * ((i >> 2) * kBlock + t) + (i & 3)); };
    uint32_t tau, r;
    if (cc < T) {
        // fewer than T keys above -inf: every key of the row counts (-inf,
        // NaN), the radix passes of select_exact run over the registers
        Radix rx;
        rx.prefix = 0;
        rx.pmask = 0;
        rx.remaining = T;
        rx.shift = 32;
        while (rx.shift > 0) {
            __syncthreads();  // (the previous pass's scan, or sm.red, has been read)
            clear_hist(sm);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kShortPer; ++i)
                if ((int32_t)pos(i) < n && rx.counts(ck[i], false)) atomicAdd(&sm.hist[rx.digit(ck[i])], 1u);
            __syncthreads();
            rx.finish(sm);
        }
        tau = rx.prefix;
        r = rx.remaining;
    } else {
        radix_tau(ck, cmax, cmin, T, sm, tau, r);
    }
#pragma unroll
    for (int i = 0; i < kShortPer; ++i)
        if ((int32_t)pos(i) < n) Ranker::mark(sm, pos(i), ck[i] > tau, ck[i] == tau);
    __syncthreads();
    Ranker::scan(sm);
    // the winners go out in batches of one load's four keys
#pragma unroll
    for (int g = 0; g < kShortPer / 4; ++g) {
        int32_t at[4];
        uint32_t cp[4], kk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * g + e;
            cp[e] = pos(i);
            kk[e] = ck[i];
            at[e] = ((int32_t)cp[e] < n && ck[i] >= tau) ? Ranker::slot(sm, cp[e], ck[i] > tau, r) : -1;
        }
        emit(at, cp, kk);
    }
    __syncthreads();
}

// ------------------------------------------------------------ key sources
// Columns [lo, lo + n) of one fp32 score row.
struct RowSrc {
    static constexpr bool kFloats = true;
    static constexpr bool kBuffer = true;
    const float* row;  // already offset by lo
    int32_t n;
    bool vec;
    // raw buffer descriptor of the n entries (loads at or past n return zeros)
    __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc() const {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), 0, n * 4, kRawDword);
    }
    // raw float bits of positions p..p+3, -inf past n
    __device__ __forceinline__ void load_raw4(int32_t p, uint32_t (&v)[4]) const {
        if (vec && p + 3 < n) {
            const float4 x = *reinterpret_cast<const float4*>(row + p);
            v[0] = __float_as_uint(x.x);
            v[1] = __float_as_uint(x.y);
            v[2] = __float_as_uint(x.z);
            v[3] = __float_as_uint(x.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = p + e < n ? __float_as_uint(row[p + e]) : kNegInfBits;
        }
    }
    __device__ __forceinline__ void load4(int32_t p, uint32_t (&k)[4]) const {
        if (vec && p + 3 < n) {
            const float4 v = *reinterpret_cast<const float4*>(row + p);
            k[0] = score_key(v.x);
            k[1] = score_key(v.y);
            k[2] = score_key(v.z);
            k[3] = score_key(v.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) k[e] = p + e < n ? score_key(row[p + e]) : 0u;
        }
    }
};

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

// v1_emit for four slots [tx0, tx0 + 4) at once: every level of the
// selected -> rt -> members -> nt chain is loaded for the four slots together,
// at indices clamped into their arrays, and v1_emit's conditions are applied
// to the loaded values afterwards, so a thread waits for four dependent loads
// instead of four per slot.  Slots at or past T are skipped.
__device__ __forceinline__ void v1_emit4(const V1Params& p, int64_t row, const RowInfo& ri, int32_t tx0,
                                         const int32_t (&raw)[4], const bool (&neg_inf)[4]) {
    int32_t page[4], logical[4], physical[4];
    bool live[4], member[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        live[i] = raw[i] >= 0 && !neg_inf[i];
        member[i] = raw[i] < ri.take * 64;
        page[i] = -1;
    }
    const int32_t last_rank = max(ri.take - 1, 0);
    if (ri.take > 0) {
        if (p.direct_fine) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                page[i] = p.fine_table[row * p.fine_table_cols + min(max(raw[i], 0) / 64, last_rank)];
        } else {
            int32_t rank[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) rank[i] = sel_rank(p, row, min(max(raw[i], 0) / 64, last_rank));
            if (p.pages > 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int32_t pg = p.rt[row * p.pages + min(max(rank[i], 0), p.pages - 1)];
                    page[i] = rank[i] >= 0 && rank[i] < p.pages ? pg : -1;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) logical[i] = -1;
    if (p.member_pages > 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int32_t m = p.members[(int64_t)min(max(page[i], 0), p.member_pages - 1) * 64 + (raw[i] & 63)];
            logical[i] = page[i] >= 0 && page[i] < p.member_pages ? m : -1;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t off = raw[i] - ri.take * 64;
        if (!member[i]) logical[i] = off < ri.sink ? off : ri.tail + off - ri.sink;
        if (!live[i]) logical[i] = -1;
        physical[i] = -1;
    }
    if (p.pages > 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = logical[i] >= 0 && logical[i] < ri.n && logical[i] / 64 < p.pages;
            const int32_t np = p.nt[row * p.pages + min(max(logical[i], 0) / 64, p.pages - 1)];
            physical[i] = ok ? np * 64 + (logical[i] & 63) : -1;
            if (!ok) logical[i] = -1;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) logical[i] = -1;
    }
    const int32_t T = p.topk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t tx = tx0 + i;
        if (tx >= T) continue;
        const int64_t dst = row * T + tx;
        p.logical[dst] = logical[i];
        if (p.physical_output) {
            p.physical[dst] = physical[i];
            p.raw[dst] = raw[i];
        }
        if (p.expansion_stride) {
            const int32_t b = logical[i] * 4;
            int4 v = logical[i] < 0 ? make_int4(-1, -1, -1, -1) : make_int4(b, b + 1, b + 2, b + 3);
            *reinterpret_cast<int4*>(p.expanded + row * p.expansion_stride + 4 * tx) = v;
        }
    }
}

// Winners staged by slot in the candidate-key array (free once the ranks are
// taken): a raw position, or a merge's workspace candidate index, with bit 31
// set for a -inf key.
constexpr uint32_t kStagedNegInf = 0x80000000u;
__device__ __forceinline__ uint32_t* v1_stage(SelSmem& sm) { return sm.cand_key; }

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

// A batch of selected items: every table entry is loaded (from a clamped
// index) before any store, so a thread's lookups overlap.  The restrict
// parameters state that the table and the outputs do not alias.
template <int N>
__device__ __forceinline__ void transform_emit_batch(const int32_t* __restrict__ table, int32_t table_cols, int bits,
                                                     int32_t* __restrict__ indices, int32_t* __restrict__ raws,
                                                     const int32_t (&at)[N], const int32_t (&raw)[N]) {
    int32_t entry[N];
#pragma unroll
    for (int i = 0; i < N; ++i) entry[i] = table_cols > 0 ? table[min(max(raw[i] >> bits, 0), table_cols - 1)] : 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (at[i] < 0) continue;
        const bool mapped = raw[i] >= 0 && (raw[i] >> bits) < table_cols;
        indices[at[i]] = mapped ? (entry[i] << bits) | (raw[i] & ((1 << bits) - 1)) : -1;
        if (raws) raws[at[i]] = raw[i];
    }
}

// Sets sm.maskpage for the ranks touching [lo, lo + span) (span <= kSpan) and
// writes -inf in place for every masked position below min(take * 64, cols)
// in that range, so the selection then reads the masked row as it lies in
// memory: the closing barrier is a work-group release / acquire, which
// orders these stores before every later load of the work-group (its waves
// share one CU and its vector L1, which stores write through).
// sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:71-107.  Ends with a barrier.
__device__ void v1_prepare_mask(const V1Params& p, int64_t row, const RowInfo& ri, int32_t lo, int32_t span, SelSmem& sm,
                                int32_t& masked_end) {
    const int t = threadIdx.x;
    const int32_t limit = min(lo + span, min(ri.take * 64, p.cols));
    masked_end = p.mask ? max(0, limit - lo) : 0;
    const int32_t nranks = (masked_end + 63) / 64;
    for (int32_t r = t; r < nranks; r += kBlock) sm.maskpage[r] = v1_mask_page(p, row, lo / 64 + r, ri);
    __syncthreads();
    float* rowp = p.scores + row * p.score_stride + lo;
    for (int32_t j = t; j < masked_end; j += kBlock) {
        const int32_t page = sm.maskpage[j >> 6];
        if (page >= 0) {
            const int32_t lg = p.members[(int64_t)page * 64 + (j & 63)];
            if (lg < ri.sink || lg >= ri.tail) rowp[j] = -__builtin_huge_valf();
        }
    }
    __syncthreads();
}

// Columns [lo, lo + n) of a V1 row, masked in place by v1_prepare_mask.
__device__ __forceinline__ RowSrc v1_source(const V1Params& p, int64_t row, int32_t lo, int32_t n) {
    const float* rp = p.scores + row * p.score_stride + lo;
    return RowSrc{rp, n, (reinterpret_cast<uintptr_t>(rp) & 15) == 0};
}

// --------------------------------------------------------- single pass
// kShortRows: every row of the call has at most kShort columns (select_short).
template <bool kShortRows>
__global__ __launch_bounds__(kBlock, 8) void v1_topk_rows(V1Params p) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const RowInfo ri = v1_row_info(p, row);
    const int32_t L = max(0, min(p.fine_lens[row], p.cols));
    int32_t masked_end;
    v1_prepare_mask(p, row, ri, 0, kSpan, sm, masked_end);
    const RowSrc src = v1_source(p, row, 0, L);
    const int32_t T = p.topk;
    if (L <= T) {
        for (int tx = threadIdx.x; tx < T; tx += kBlock) {
            bool inf = false;
            if (tx < L) {
                uint32_t k[4];
                src.load4(tx & ~3, k);
                inf = k[tx & 3] == kNegInfKey;
            }
            v1_emit(p, row, ri, tx, tx < L ? tx : -1, inf);
        }
    } else {
        uint32_t* stage = v1_stage(sm);
        auto emit = [&](const auto& at, const auto& pos, const auto& key) {
#pragma unroll
            for (int i = 0; i < (int)(sizeof(at) / sizeof(at[0])); ++i)
                if (at[i] >= 0) stage[at[i]] = (uint32_t)pos[i] | (key[i] == kNegInfKey ? kStagedNegInf : 0u);
        };
        if constexpr (kShortRows)
            select_short(src, (uint32_t)T, sm, emit);
        else
            select_stream(src, (uint32_t)T, sm, emit);
        // (the selection ends with a barrier: every slot is staged)
        for (int32_t tx0 = 4 * threadIdx.x; tx0 < T; tx0 += 4 * kBlock) {
            int32_t raw[4];
            bool inf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t v = tx0 + i < T ? stage[tx0 + i] : 0u;
                raw[i] = (int32_t)(v & ~kStagedNegInf);
                inf[i] = (v & kStagedNegInf) != 0;
            }
            v1_emit4(p, row, ri, tx0, raw, inf);
        }
    }
    v1_pad_expansion(p, row);
}

template <bool kShortRows>
__global__ __launch_bounds__(kBlock, 8) void transform_rows(TransformParams p) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    const int32_t T = p.topk;
    if (L <= T) {
        for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, tx < L ? tx : -1);
        return;
    }
    const float* rp = p.scores + row * p.score_stride;
    const RowSrc src{rp, L, (reinterpret_cast<uintptr_t>(rp) & 15) == 0};
    const int32_t* table = p.page_table + row * p.page_table_stride;
    int32_t* out = p.page_indices + row * p.topk;
    int32_t* raws = p.raw_indices ? p.raw_indices + row * p.topk : nullptr;
    // Pages of at least 64 positions: the row's page table (at most
    // kSpan / 64 <= 2 kBlock entries) is staged in LDS (the mask-page array,
    // unused by plain rows), its loads issued with the pivot sample's.
    const int bits = p.page_bits;
    const bool staged = bits >= kTableBits;
    const int32_t entries = staged ? min(p.page_table_cols, kSpan >> bits) : 0;
    const int32_t entry = (int32_t)threadIdx.x < entries ? table[threadIdx.x] : 0;
    const int32_t entry2 = (int32_t)threadIdx.x + kBlock < entries ? table[threadIdx.x + kBlock] : 0;
    static_assert(kSpan / 64 <= 2 * kBlock, "two table entries per thread");
    auto emit = [&](const auto& at, const auto& pos, const auto&) {
        constexpr int N = sizeof(at) / sizeof(at[0]);
        int32_t raw[N];
#pragma unroll
        for (int i = 0; i < N; ++i) raw[i] = (int32_t)pos[i];
        if (staged) {
            // slot -> position into LDS (the candidate-key array: read only
            // before the ranks); written out in slot order below
            uint16_t* stage = reinterpret_cast<uint16_t*>(sm.cand_key);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (at[i] >= 0) stage[at[i]] = (uint16_t)raw[i];
        } else {
            transform_emit_batch<N>(table, p.page_table_cols, bits, out, raws, at, raw);
        }
    };
    if constexpr (kShortRows) {
        if (staged) {  // read after select_short's first barrier
            sm.maskpage[threadIdx.x] = entry;
            if ((int32_t)threadIdx.x + kBlock < kSpan / 64) sm.maskpage[threadIdx.x + kBlock] = entry2;
        }
        select_short(src, (uint32_t)T, sm, emit);
    } else {
        uint32_t sk[4];
        src.load4(sample_pos(L), sk);
        if (staged) {  // read after select_sampled's first barrier
            sm.maskpage[threadIdx.x] = entry;
            if ((int32_t)threadIdx.x + kBlock < kSpan / 64) sm.maskpage[threadIdx.x + kBlock] = entry2;
        }
        select_sampled(src, sk, (uint32_t)T, sm, emit);
    }
    if (!staged) return;
    // (the selection ends with a barrier: every slot is staged) slots in
    // order, four per thread and 16-byte stores where the rows allow them
    const uint16_t* stage = reinterpret_cast<const uint16_t*>(sm.cand_key);
    const int32_t lo_mask = (1 << bits) - 1;
    auto map = [&](int32_t raw) {
        const int32_t e = raw >> bits;
        return e < entries ? (sm.maskpage[e] << bits) | (raw & lo_mask) : -1;
    };
    const bool vec = T % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(raws) & 15) == 0;
    if (vec) {
        for (int32_t q = threadIdx.x; q < T / 4; q += kBlock) {
            const uint2 w2 = *reinterpret_cast<const uint2*>(stage + 4 * q);
            const int32_t r0 = (int32_t)(w2.x & 0xffffu), r1 = (int32_t)(w2.x >> 16);
            const int32_t r2 = (int32_t)(w2.y & 0xffffu), r3 = (int32_t)(w2.y >> 16);
            *reinterpret_cast<int4*>(out + 4 * q) = make_int4(map(r0), map(r1), map(r2), map(r3));
            if (raws) *reinterpret_cast<int4*>(raws + 4 * q) = make_int4(r0, r1, r2, r3);
        }
    } else {
        for (int32_t tx = threadIdx.x; tx < T; tx += kBlock) {
            const int32_t raw = stage[tx];
            out[tx] = map(raw);
            if (raws) raws[tx] = raw;
        }
    }
}

// ------------------------------------------------------- segmented rows
// Workspace per (row, segment): T keys, T positions, then one count per pair.
struct Workspace {
    uint32_t* keys;
    int32_t* pos;
    int32_t* count;
    int32_t nseg;
    int32_t seg;  // columns per segment (a multiple of 64, <= kSpan)
    int32_t T;
    __device__ __forceinline__ int64_t at(int64_t row, int32_t s) const { return (row * nseg + s) * (int64_t)T; }
};

// Segments of a row: the fewest that keep each within segment_span columns
// (more segments make the merge, which selects over nseg * topk candidates,
// cost as much as they save).  One segment means the single-pass kernel.
struct SegPlan {
    int32_t nseg, seg;
};
// Longest segment: the work-group's whole span for batches of 512 rows or
// more; 32768 columns below, where more, shorter segments keep more of the
// GPU busy.  Measured: 1024 rows of 34880 columns in one pass 57 us against
// 108 us as two segments and a merge; 128 rows of up to 67K columns 48 us as
// three segments of at most 32768 columns against 51 us as two.
inline int64_t segment_span(int32_t batch) { return batch >= 512 ? kSpan : 32768; }
inline SegPlan plan_segments(int32_t batch, int32_t cols, int32_t topk) {
    (void)topk;
    const int64_t nseg = cdiv(cols, segment_span(batch));
    if (nseg <= 1) return SegPlan{1, cols};
    const int64_t seg = cdiv(cdiv(cols, nseg), 64) * 64;
    return SegPlan{(int32_t)cdiv(cols, seg), (int32_t)seg};
}

inline int64_t workspace_bytes(int32_t batch, const SegPlan& plan, int32_t topk) {
    return plan.nseg > 1 ? (int64_t)batch * plan.nseg * ((int64_t)topk * 8 + 4) : 0;
}

inline Workspace make_workspace(void* base, int32_t batch, const SegPlan& plan, int32_t topk) {
    Workspace ws;
    ws.nseg = plan.nseg;
    ws.seg = plan.seg;
    ws.T = topk;
    const int64_t pairs = (int64_t)batch * ws.nseg;
    ws.keys = static_cast<uint32_t*>(base);
    ws.pos = reinterpret_cast<int32_t*>(ws.keys + pairs * topk);
    ws.count = ws.pos + pairs * topk;
    return ws;
}

// Segment s of a row: its Top-T (all of it when shorter) into the workspace in
// ascending position.  Keys are forced >= 1 so that the merge's padding key 0
// stays strictly below every real candidate.
template <class Src>
__device__ __forceinline__ void segment_select(const Src& src, int32_t lo, int32_t T, const Workspace& ws, int64_t row,
                                               int32_t s, SelSmem& sm) {
    const int64_t at = ws.at(row, s);
    const int32_t n = src.n;
    if (n <= T) {
        for (int32_t j = 4 * threadIdx.x; j < n; j += 4 * kBlock) {
            uint32_t k[4];
            src.load4(j, k);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (j + e < n) {
                    ws.keys[at + j + e] = max(k[e], 1u);
                    ws.pos[at + j + e] = lo + j + e;
                }
            }
        }
        if (threadIdx.x == 0) ws.count[row * ws.nseg + s] = n;
        return;
    }
    select_stream(src, (uint32_t)T, sm, [&](const auto& slot, const auto& pos, const auto& key) {
#pragma unroll
        for (int i = 0; i < (int)(sizeof(slot) / sizeof(slot[0])); ++i) {
            if (slot[i] < 0) continue;
            ws.keys[at + slot[i]] = max(key[i], 1u);
            ws.pos[at + slot[i]] = lo + (int32_t)pos[i];
        }
    });
    if (threadIdx.x == 0) ws.count[row * ws.nseg + s] = T;
}

__global__ __launch_bounds__(kBlock, 8) void v1_topk_segments(V1Params p, Workspace ws) {
    __shared__ SelSmem sm;
    const int32_t s = blockIdx.x;
    const int64_t row = blockIdx.y;
    const RowInfo ri = v1_row_info(p, row);
    const int32_t L = max(0, min(p.fine_lens[row], p.cols));
    const int32_t lo = s * ws.seg;
    int32_t masked_end;
    v1_prepare_mask(p, row, ri, lo, ws.seg, sm, masked_end);
    if (L <= p.topk) return;  // the merge kernel takes every candidate
    const int32_t n = max(0, min(L - lo, ws.seg));
    segment_select(v1_source(p, row, lo, n), lo, p.topk, ws, row, s, sm);
}

__global__ __launch_bounds__(kBlock, 8) void transform_segments(TransformParams p, Workspace ws) {
    __shared__ SelSmem sm;
    const int32_t s = blockIdx.x;
    const int64_t row = blockIdx.y;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    if (L <= p.topk) return;
    const int32_t lo = s * ws.seg;
    const int32_t n = max(0, min(L - lo, ws.seg));
    const float* rp = p.scores + row * p.score_stride + lo;
    segment_select(RowSrc{rp, n, (reinterpret_cast<uintptr_t>(rp) & 15) == 0}, lo, p.topk, ws, row, s, sm);
}

// The concatenated segment candidates of a row: position q = s*T + k.
struct CandSrc {
    static constexpr bool kFloats = false;
    static constexpr bool kBuffer = false;
    const uint32_t* keys;  // workspace keys of this row
    const int32_t* count;  // per segment
    int32_t T;
    int32_t nseg;
    int32_t n;
    __device__ __forceinline__ void load_raw4(int32_t q, uint32_t (&k)[4]) const { load4(q, k); }
    __device__ __forceinline__ void load4(int32_t q, uint32_t (&k)[4]) const {
        if ((T & 3) == 0) {
            // q % 4 == 0: the four entries lie in one segment's list, which
            // starts 16-byte aligned
            const int32_t s = q / T, j = q - s * T;
            const int32_t c = s < nseg ? count[s] : 0;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (j < c) v = *reinterpret_cast<const uint4*>(keys + q);
            k[0] = j < c ? v.x : 0u;
            k[1] = j + 1 < c ? v.y : 0u;
            k[2] = j + 2 < c ? v.z : 0u;
            k[3] = j + 3 < c ? v.w : 0u;
            return;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int32_t qq = q + e;
            const int32_t s = qq / T, j = qq - s * T;
            k[e] = (s < nseg && j < count[s]) ? keys[qq] : 0u;
        }
    }
};

__device__ __forceinline__ CandSrc cand_source(const Workspace& ws, int64_t row) {
    return CandSrc{ws.keys + ws.at(row, 0), ws.count + row * ws.nseg, ws.T, ws.nseg, ws.nseg * ws.T};
}

// kShortMerge: the segments' candidates (nseg * T) fit kShort (select_short);
// one work-group per row, so that instance may take more registers than the
// 64 that four work-groups per CU allow.
template <bool kShortMerge>
__global__ __launch_bounds__(kBlock, kShortMerge ? 4 : 8) void v1_topk_merge(V1Params p, Workspace ws) {
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
    } else if (L <= ws.seg) {
        // one non-empty segment: its list is the row's Top-T in position order
        const int32_t* pos = ws.pos + ws.at(row, 0);
        const uint32_t* keys = ws.keys + ws.at(row, 0);
        for (int32_t tx0 = 4 * threadIdx.x; tx0 < T; tx0 += 4 * kBlock) {
            int32_t raw[4];
            bool inf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int32_t tx = min(tx0 + i, T - 1);
                raw[i] = pos[tx];
                inf[i] = keys[tx] == kNegInfKey;
            }
            v1_emit4(p, row, ri, tx0, raw, inf);
        }
    } else {
        const int32_t* pos = ws.pos + ws.at(row, 0);
        uint32_t* stage = v1_stage(sm);
        auto emit = [&](const auto& at, const auto& q, const auto& key) {
#pragma unroll
            for (int i = 0; i < (int)(sizeof(at) / sizeof(at[0])); ++i)
                if (at[i] >= 0) stage[at[i]] = (uint32_t)q[i] | (key[i] == kNegInfKey ? kStagedNegInf : 0u);
        };
        if constexpr (kShortMerge)
            select_short(cand_source(ws, row), (uint32_t)T, sm, emit);
        else
            select_stream(cand_source(ws, row), (uint32_t)T, sm, emit);
        // (the selection ends with a barrier: every slot holds a candidate index)
        for (int32_t tx0 = 4 * threadIdx.x; tx0 < T; tx0 += 4 * kBlock) {
            int32_t raw[4];
            bool inf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t v = stage[min(tx0 + i, T - 1)];
                raw[i] = pos[min(v & ~kStagedNegInf, (uint32_t)(ws.nseg * T - 1))];
                inf[i] = (v & kStagedNegInf) != 0;
            }
            v1_emit4(p, row, ri, tx0, raw, inf);
        }
    }
    v1_pad_expansion(p, row);
}

template <bool kShortMerge>
__global__ __launch_bounds__(kBlock, 8) void transform_merge(TransformParams p, Workspace ws) {
    __shared__ SelSmem sm;
    const int64_t row = blockIdx.x;
    const int32_t L = max(0, min(p.seq_lens[row], p.cols));
    const int32_t T = p.topk;
    if (L <= T) {
        for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, tx < L ? tx : -1);
        return;
    }
    const int32_t* pos = ws.pos + ws.at(row, 0);
    if (L <= ws.seg) {
        // one non-empty segment: its list is the row's Top-T in position order
        for (int tx = threadIdx.x; tx < T; tx += kBlock) transform_emit(p, row, tx, pos[tx]);
        return;
    }
    const int32_t nq = ws.nseg * T;
    auto emit = [&](const auto& at, const auto& q, const auto&) {
        constexpr int N = sizeof(at) / sizeof(at[0]);
        int32_t raw[N];
#pragma unroll
        for (int i = 0; i < N; ++i) raw[i] = pos[min((int32_t)q[i], nq - 1)];
        transform_emit_batch<N>(p.page_table + row * p.page_table_stride, p.page_table_cols, p.page_bits,
                                p.page_indices + row * p.topk, p.raw_indices ? p.raw_indices + row * p.topk : nullptr,
                                at, raw);
    };
    if constexpr (kShortMerge)
        select_short(cand_source(ws, row), (uint32_t)T, sm, emit);
    else
        select_stream(cand_source(ws, row), (uint32_t)T, sm, emit);
}

// ------------------------------------------------------ unfused mask/map
// sglang/srt/layers/attention/v1_deepseek/kernels.py:444-472.
// One thread per 4 consecutive columns (they share one 64-column page, so
// its rank, table entry and 4 members come from 3 loads); only columns that
// are masked are written.
__global__ __launch_bounds__(256) void mask_fine_kernel(float* scores, int64_t stride, const void* selected,
                                                        int32_t sel64, const int32_t* rt, const int32_t* members,
                                                        const int32_t* lens, const int32_t* takes, int32_t maxp,
                                                        int32_t take_stride, int32_t width, int32_t sink_cap,
                                                        int32_t window, int32_t vec) {
    const int64_t row = blockIdx.y;
    const int32_t j0 = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (j0 >= width) return;
    const int32_t n = lens[row];
    const int32_t take = takes[row];
    const int32_t sink = min(n, sink_cap);
    const int32_t tail = max(sink, min(max(n - 1, 0) / 1024 * 1024, max(sink, n - window)));
    const int32_t count = take * 64 + sink + n - tail;
    const bool fine = j0 < take * 64;  // (take * 64 is a multiple of 4: the 4 columns agree)
    int4 lg = make_int4(-1, -1, -1, -1);
    if (fine && j0 / 64 < take_stride) {
        const int32_t rank = sel64 ? (int32_t) static_cast<const int64_t*>(selected)[row * take_stride + j0 / 64]
                                   : static_cast<const int32_t*>(selected)[row * take_stride + j0 / 64];
        if (rank >= 0 && rank < maxp) {
            const int32_t page = rt[row * maxp + rank];
            if (page >= 0) {
                const int32_t* m = members + (int64_t)page * 64 + (j0 & 63);
                lg = vec ? *reinterpret_cast<const int4*>(m) : make_int4(m[0], m[1], m[2], m[3]);
            }
        }
    }
    const int32_t l4[4] = {lg.x, lg.y, lg.z, lg.w};
    float* out = scores + row * stride + j0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int32_t j = j0 + e;
        const bool good = j < count && (!fine || (l4[e] >= sink && l4[e] < tail));
        if (j < width && !good) out[e] = -__builtin_huge_valf();
    }
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
int launch_topk(void (*single)(P), void (*single_short)(P), void (*seg)(P, Workspace), void (*merge)(P, Workspace),
                void (*merge_short)(P, Workspace), int32_t cols, int32_t batch, int32_t topk, void* wsp,
                int64_t ws_bytes, const P& p, hipStream_t st, const char* name) {
    const SegPlan plan = plan_segments(batch, cols, topk);
    const int64_t need = workspace_bytes(batch, plan, topk);
    // rows within one work-group's span also run in one pass when the caller
    // gives no (or too small a) workspace for the split; calls whose rows
    // all fit kShort columns hold each row in registers
    if (plan.nseg == 1 || (cols <= kSpan && (wsp == nullptr || ws_bytes < need))) {
        hipLaunchKernelGGL(cols <= kShort ? single_short : single, dim3(batch), dim3(kBlock), 0, st, p);
        return V1_LAUNCHED(name);
    }
    V1_REQUIRE(wsp != nullptr && ws_bytes >= need, "%s: rows longer than %d columns need a workspace of %lld bytes",
               name, kSpan, (long long)need);
    V1_REQUIRE((reinterpret_cast<uintptr_t>(wsp) & 15) == 0, "%s: the workspace must be 16-byte aligned", name);
    const Workspace ws = make_workspace(wsp, batch, plan, topk);
    V1_REQUIRE((int64_t)ws.nseg * topk <= kSpan, "%s: %d columns exceed the %lld supported at topk %d", name, cols,
               (long long)(kSpan / topk) * segment_span(batch), topk);
    hipLaunchKernelGGL(seg, dim3(ws.nseg, batch), dim3(kBlock), 0, st, p, ws);
    int rc = V1_LAUNCHED(name);
    if (rc != V1_OK) return rc;
    hipLaunchKernelGGL((int64_t)ws.nseg * topk <= kShort ? merge_short : merge, dim3(batch), dim3(kBlock), 0, st, p,
                       ws);
    return V1_LAUNCHED(name);
}

// kernels.py:594-600 (expand_logical): out[row, j] = 4 * logical[row, j / 4]
// + j % 4 for j < 4 * topk with a valid (>= 0) index, else -1, for j < cols;
// rows of out are `stride` ints apart.  One thread per 4 output ints;
// int32 arithmetic wraps as the reference's does.
__global__ __launch_bounds__(256) void expand_logical_kernel(const int32_t* __restrict__ logical,
                                                             int32_t* __restrict__ out, int32_t topk,
                                                             int64_t stride, int32_t cols, int32_t vec) {
    const int64_t row = blockIdx.y;
    const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * (int64_t)i >= cols) return;
    const int32_t v = i < topk ? logical[row * topk + i] : -1;
    const uint32_t base = (uint32_t)v * 4u;
    const int4 r = v >= 0 ? make_int4((int32_t)base, (int32_t)(base + 1), (int32_t)(base + 2), (int32_t)(base + 3))
                          : make_int4(-1, -1, -1, -1);
    int32_t* dst = out + row * stride + 4 * (int64_t)i;
    if (vec) {
        *reinterpret_cast<int4*>(dst) = r;
    } else {
        const int32_t n = cols - 4 * i < 4 ? cols - 4 * i : 4;
        dst[0] = r.x;
        if (n > 1) dst[1] = r.y;
        if (n > 2) dst[2] = r.z;
        if (n > 3) dst[3] = r.w;
    }
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int64_t v1_topk_workspace(int32_t batch, int32_t cols, int32_t topk) {
    if (batch <= 0 || topk <= 0 || cols <= 0) return 0;
    return workspace_bytes(batch, plan_segments(batch, cols, topk), topk);
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
    return launch_topk<V1Params>(v1_topk_rows<false>, v1_topk_rows<true>, v1_topk_segments, v1_topk_merge<false>,
                                 v1_topk_merge<true>, a->cols, a->batch, a->topk,
                                 a->workspace, a->workspace_bytes, p, as_stream(stream), "v1_topk");
}

extern "C" int v1_topk_transform(const v1_topk_transform_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "topk_transform: null args");
    V1_REQUIRE(a->batch >= 0 && a->cols >= 0, "topk_transform: bad shape");
    V1_REQUIRE(a->topk > 0 && a->topk <= V1_MAX_TOPK, "topk_transform: topk must be in (0, 2048]");
    V1_REQUIRE(a->page_bits >= 0 && a->page_bits < 31, "topk_transform: bad page_bits");
    if (a->batch == 0) return V1_OK;
    TransformParams p{a->scores, a->score_stride, a->cols, a->seq_lens, a->page_table, a->page_table_stride,
                      a->page_table_cols, a->page_bits, a->page_indices, a->raw_indices, a->topk};
    return launch_topk<TransformParams>(transform_rows<false>, transform_rows<true>, transform_segments,
                                        transform_merge<false>, transform_merge<true>, a->cols, a->batch,
                                        a->topk, a->workspace, a->workspace_bytes, p, as_stream(stream),
                                        "topk_transform");
}

extern "C" int v1_mask_fine(float* scores, int64_t score_stride, const void* selected, int32_t selected_bits,
                            const int32_t* rt, const int32_t* members, const int32_t* lens, const int32_t* takes,
                            int32_t rows, int32_t maxp, int32_t take_stride, int32_t width, int32_t sink,
                            int32_t window, void* stream) {
    V1_REQUIRE(rows >= 0 && width >= 0 && maxp > 0, "mask_fine: bad shape");
    V1_REQUIRE(selected_bits == 32 || selected_bits == 64, "mask_fine: selected must be int32 or int64");
    if (rows == 0 || width == 0) return V1_OK;
    const int32_t vec = (reinterpret_cast<uintptr_t>(members) & 15) == 0 ? 1 : 0;
    hipLaunchKernelGGL(mask_fine_kernel, dim3((uint32_t)cdiv(width, 1024), rows), dim3(256), 0, as_stream(stream),
                       scores, score_stride, selected, selected_bits == 64, rt, members, lens, takes, maxp,
                       take_stride, width, sink, window, vec);
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

extern "C" int v1_expand_logical(const int32_t* logical, int32_t* out, int32_t rows, int32_t topk, int64_t stride,
                                 int32_t cols, void* stream) {
    V1_REQUIRE(rows >= 0 && topk >= 0 && cols >= 0 && stride >= cols, "expand_logical: bad shape");
    if (rows == 0 || cols == 0) return V1_OK;
    const int32_t vec = (cols % 4 == 0 && stride % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) ? 1 : 0;
    hipLaunchKernelGGL(expand_logical_kernel, dim3((uint32_t)cdiv(cdiv(cols, 4), 256), rows), dim3(256), 0,
                       as_stream(stream), logical, out, topk, stride, cols, vec);
    return V1_LAUNCHED("expand_logical");
}
