// FP8 paged MQA index logits on CDNA4 MFMA (v_mfma_f32_16x16x128_f8f6f4):
//   logits[r, j] = sum_h w[r,h] * ReLU(sum_d q[r,h,d] * k[j,d]) * s_k[j]
// Formula: sglang/srt/layers/attention/v1_deepseek/kernels.py:248-320 and
// experiments/fine_pool_shared_20261021/test_and_bench.py:37; the DeepGEMM
// fp8_paged_mqa_logits call sites are runtime.py:434-444, 538-548.
//
// One MFMA multiplies 16 heads x 128 dims of a query by 16 keys x 128 dims:
// lane l holds 32 FP8 bytes of head (l%16) / key (l%16) at dims 32*(l/16)..+32
// for A / B (any consistent dim split gives the same dot product), and the
// 16x16 fp32 result D[4*(l/16)+i][l%16] in its 4 accumulators.  The head
// weighting is done per lane (16 heads of a 64-head query per lane group),
// then folded across the 4 lane groups with two xor shuffles, which leaves
// the logit of key l%16 in every lane group; the group whose index matches the
// 16-key block keeps it, so a 64-key page ends as one logit per lane and is
// stored with one coalesced 256-byte write.
//
// Shared-table rows (a prefill chunk of one request) are tiled 8 queries per
// work-group: each 8448-byte key page is staged once in LDS (chunks of each
// key row swizzled so that the 16-byte fragment reads are bank-conflict free)
// and reused by 8 queries x 64 heads.  Rows with their own tables run one
// query per work-group, each wave streaming whole pages straight from HBM
// (decode batches), or, for more than 512 rows of more than 16 heads (a
// prefill chunk's rows share most of their pages), through the same LDS page
// ring over the union of each 8-row group's table pages (score_union_plan +
// the union form of score_shared), each wave skipping the pages none of its
// queries lists.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace v1 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
// Word 3 of a raw buffer descriptor (stride 0, 32-bit dwords).  Accesses at
// byte offsets at or past the descriptor's length are range-checked by the
// hardware: loads return zeros and stores are dropped.
constexpr int32_t kRawDword = 0x00020000;
constexpr int kChunkPages = 16;                      // pages per work-group
constexpr int kQueriesPerWave = 2;
constexpr int kQueriesPerGroup = 4 * kQueriesPerWave;

__device__ __forceinline__ v4f mfma_fp8(v8i a, v8i b) {
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

struct ScoreParams {
    const uint8_t* q;
    const uint8_t* kv;
    int64_t kv_blocks;
    const float* w;
    const int32_t* ctx;
    const int32_t* table;
    int64_t table_stride;
    int32_t max_blocks;
    float* logits;
    int64_t logits_stride;
    int32_t max_context_len;
    int32_t rows;
    int32_t heads;
    int32_t relu;
    int32_t clean;
    const uint8_t* pieces;  // per-query records from score_prep (shared-table kernel)
    int32_t nchunks;        // shared-table kernel: chunks of kChunkPages pages over max_context_len
    int32_t groups;         // shared-table kernel: 8-query row groups
    int32_t items;          // shared-table kernel: groups x levels
    uint32_t* work;         // shared-table kernel: next work item (zeroed by score_prep)
    int32_t bulk;           // shared-table kernel: levels of full-size ranges (chunks [L*F, (L+1)*F))
    int32_t full;           // shared-table kernel: F, the chunks of a full-size range
    int32_t lvl_start[16];  // shared-table kernel: chunk range of each later level's items
    int32_t lvl_chunks[16];
    uint32_t* exact_pages;  // shared-table ReLU path: per row, a bitmap of pages for score_exact
    int32_t exact_words;    // 32-bit words per row of exact_pages (score_exact)
    // union form (per-row tables through the page ring), built by score_union_plan:
    const int32_t* u_pages;    // [groups * u_cap] pool page of each union entry (-1: none, reads zeros)
    const uint32_t* u_mask;    // [groups * u_cap] rows of the group that list the entry (bit q)
    const int32_t* u_slots;    // [groups * u_cap * 8] the table slot of row q (where its mask bit is set)
    const int32_t* u_items;    // [kUnionLevels * u_level_stride] (group, first entry | entries << 16)
    const int32_t* u_level_n;  // [kUnionLevels] items per level
    int32_t u_cap;             // union entries per group (8 * table pages of max_context_len)
    int32_t u_level_stride;
    const int32_t* row_filter;  // score_rows: rows whose entry is 0 are skipped (nullptr: every row)
};
constexpr int kMaxLevels = 16;

// ---------------------------------------------------------- linear term
// relu(x) = (x + |x|) / 2, so  sum_h w_h relu(q_h . k)
//   = 1/2 (sum_h w_h q_h) . k  +  1/2 sum_h w_h |q_h . k|.
// The first term is one more dot product per query: q' = sum_h w_h q_h is
// split into kPieces FP8 (e4m3fn) vectors with power-of-two scales,
// q' ~= sum_p s_p u_p, each piece taking the residual of the previous ones
// (every piece shrinks the residual at least 16x, so the last one leaves
// less than 16^-8 of max|q'|), and those pieces ride in an MFMA row block.
constexpr int kPieces = 8;
// Per-query record written by score_prep for the shared-table kernel:
//   [0, 1024)     kPieces x 128 FP8 piece bytes
//   [1024, 1056)  kPieces fp32 piece scales, times 1/2 (the linear-term factor)
//   [1056, 1312)  64 fp32 head weights, times 1/2 on the ReLU path, zero past `heads`
//   [1312, 1328)  fp32 exact-path threshold (see below), then padding
// so the kernel reads everything with unconditional 16-byte loads.
constexpr int kRecScales = kPieces * 128;
constexpr int kRecWeights = kRecScales + kPieces * 4;
constexpr int kRecBound = kRecWeights + 64 * 4;
constexpr int64_t kPieceRowBytes = kRecBound + 16;
static_assert(kRecWeights % 16 == 0 && kRecBound % 16 == 0 && kPieceRowBytes % 16 == 0,
              "16-byte aligned record fields");

// Exact zeros.  The reference's sum of w * ReLU(x) is exactly 0 for a key
// whose every head dot is <= 0 (kernels.py:310-313); the linear + |x| form
// gives the difference of two separately rounded sums there instead.  Any FP8
// key has |k_d| <= 448, so every head dot obeys |q_h . k| <= 448 ||q_h||_1 and
// every fp32 rounding of the fast form (the pieces' and head MFMAs'
// 128-product sums, the head folds) is at most ~2^-15 of
//   B = 448 * sum_h |w_h| ||q_h||_1.
// A key whose fast value lies within kExactFrac * B of zero (eight times that
// worst case) is therefore recomputed the direct way, sum_h w_h * max(x_h, 0)
// in fp32, which is exactly 0 when no head dot is positive.  Keys of many
// heads with unrelated signs are never that close to zero; few live heads put
// about 2^-H of the keys on the exact path.
constexpr float kExactFrac = 1.0f / 4096.0f;

// Reductions over a wave: a DPP butterfly within each row of 16 lanes, then
// the four row results read out and combined; the result is wave-uniform.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}

template <typename Op>
__device__ __forceinline__ float wave_all(float v, Op op) {
    v = op(v, dpp_mov<0xb1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_mov<0x4e>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_mov<0x141>(v));  // row_half_mirror: the other quad of the half row
    v = op(v, dpp_mov<0x140>(v));  // row_mirror: the other half row
    auto row = [&](int lane) __attribute__((always_inline)) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    };
    return op(op(row(0), row(16)), op(row(32), row(48)));
}

// One wave per query row: q' = sum_h w_h q_h split into its pieces, and the
// record described above.  relu: 1 the fold (halved weights, pieces, the
// exact-path threshold); 0 (no ReLU) or 2 (ReLU taken directly, one head
// block) the weights alone.
__global__ __launch_bounds__(256) void score_prep(const uint8_t* q, const float* w, int32_t rows, int32_t heads,
                                                  int32_t relu, uint8_t* out, uint32_t* work, uint32_t* exact_pages,
                                                  int32_t exact_words, uint32_t* clear, int32_t nclear) {
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int l = __lane_id();
    if (blockIdx.x == 0 && threadIdx.x == 0) *work = 0u;  // the work counter of score_shared
    if (blockIdx.x == 0 && (int)threadIdx.x < nclear) clear[threadIdx.x] = 0u;  // the union plan's level counts
    if (row >= rows) return;
    for (int k = l; k < exact_words; k += kWave) exact_pages[row * exact_words + k] = 0u;
    // lane l owns dims 2l, 2l+1; every head's two bytes come in one round
    // trip of buffer loads over the query row (heads past `heads` read as
    // zeros), lane h holds head h's weight, and the sums run in head order.
    // v_cvt_pk_f32_fp8 decodes OCP e4m3fn exactly (NaN codes to NaN).
    float a0 = 0.f, a1 = 0.f, bound = 0.f;
    const float wl = w[row * heads + min(l, heads - 1)];
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(q + row * heads * 128), 0, heads * 128,
                                                      kRawDword);
    uint32_t b[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) b[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, 2 * l, j * 128, 0);
#pragma unroll
    for (int j = 0; j < 64; ++j) {
        const float wh = j < heads ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j))
                                   : 0.f;
        const auto x = __builtin_amdgcn_cvt_pk_f32_fp8((int)b[j], false);
        a0 = fmaf(wh, x[0], a0);
        a1 = fmaf(wh, x[1], a1);
        bound = fmaf(fabsf(wh), fabsf(x[0]) + fabsf(x[1]), bound);
    }
    bound = wave_all(bound, [](float x, float y) { return x + y; });
    uint8_t* dst = out + row * kPieceRowBytes;
    for (int pc = 0; pc < (relu == 1 ? kPieces : 0); ++pc) {
        const float m = wave_all(fmaxf(fabsf(a0), fabsf(a1)), [](float x, float y) { return fmaxf(x, y); });
        // scale: smallest power of two >= m / 448 (1 when the residual is zero)
        float sc = 1.f;
        if (m > 0.f) {
            int e;
            const float f = frexpf(m / 448.f, &e);  // m/448 = f * 2^e
            sc = __builtin_ldexpf(1.f, f == 0.5f ? e - 1 : e);
        }
        const uint32_t c0 = e4m3_code(a0 / sc), c1 = e4m3_code(a1 / sc);
        *reinterpret_cast<uint16_t*>(dst + pc * 128 + 2 * l) = (uint16_t)(c0 | (c1 << 8));
        if (l == 0) reinterpret_cast<float*>(dst + kRecScales)[pc] = 0.5f * sc;
        a0 -= sc * e4m3_value(c0);
        a1 -= sc * e4m3_value(c1);
    }
    reinterpret_cast<float*>(dst + kRecWeights)[l] = l < heads ? (relu == 1 ? 0.5f : 1.f) * w[row * heads + l] : 0.f;
    if (l < 4) reinterpret_cast<float*>(dst + kRecBound)[l] = l == 0 ? kExactFrac * 448.f * bound : 0.f;
}

// Prologue loads are issued unconditionally, from indices clamped into range,
// and zeroed afterwards by a select: a load inside a branch is waited for
// before the branch joins, which would serialise every one of them.

// A fragments (HB row blocks of 16 heads) of one query; zero past `heads`.
template <int HB>
__device__ __forceinline__ void load_q(const ScoreParams& p, int64_t row, v8i (&a)[HB]) {
    const int l = __lane_id();
    const int64_t rc = min(row, (int64_t)p.rows - 1);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
        const int h = hb * 16 + (l & 15);
        const bool ok = (row < p.rows) & (h < p.heads);
        const u32x4* src = reinterpret_cast<const u32x4*>(p.q + (rc * p.heads + min(h, p.heads - 1)) * 128 + 32 * (l >> 4));
        const u32x4 x = src[0], y = src[1];
        a[hb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
        if (!ok) a[hb] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    }
}

// Weights of the 4 heads (per row block) whose results this lane holds.
template <int HB>
__device__ __forceinline__ void load_w(const ScoreParams& p, int64_t row, float (&w)[HB][4]) {
    const int l = __lane_id();
    const int64_t rc = min(row, (int64_t)p.rows - 1);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = hb * 16 + 4 * (l >> 4) + i;
            const float v = p.w[rc * p.heads + min(h, p.heads - 1)];
            w[hb][i] = ((row < p.rows) & (h < p.heads)) ? v : 0.f;
        }
}

// ReLU as an integer max on the bit pattern: negative floats (and -0.0) have
// the sign bit set and compare below 0 as int32; no NaN canonicalisation.
__device__ __forceinline__ float relu(float x) {
    return __builtin_bit_cast(float, max(__builtin_bit_cast(int, x), 0));
}

// Per-lane partial logits of one query for the 4 key blocks of a page:
// s[kb] = sum over this lane's 4 heads per row block of w * relu(q . k).
template <int HB, bool RELU>
__device__ __forceinline__ void page_partials(const v8i (&a)[HB], const v8i (&b)[4], const float (&w)[HB][4],
                                              float (&s)[4]) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        float acc = 0.f;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const v4f d = mfma_fp8(a[hb], b[kb]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = fmaf(w[hb][i], RELU ? relu(d[i]) : d[i], acc);
        }
        s[kb] = acc;
    }
}

// page_partials as one stream: MFMA idx (key block idx / HB, head block
// idx % HB) goes to a ring of kLag + 1 result sets and is folded kLag MFMAs
// after issue, so the MFMA pipe works while the VALU folds older results
// (left alone, the compiler folds each result right after its MFMA and
// waits for it).  The same products in the same order as page_partials:
// the values are equal bit for bit.
template <int HB, bool RELU>
__device__ __forceinline__ void page_partials_lag(const v8i (&a)[HB], const v8i (&b)[4], const float (&w)[HB][4],
                                                  float (&s)[4]) {
    constexpr int kN = 4 * HB, kLag = 3;
    v4f d[kLag + 1];
#pragma unroll
    for (int idx = 0; idx < kN + kLag; ++idx) {
        if (idx < kN) d[idx % (kLag + 1)] = mfma_fp8(a[idx % HB], b[idx / HB]);
        const int j = idx - kLag;
        if (j >= 0) {
            const v4f x = d[j % (kLag + 1)];
            const int kb = j / HB, hb = j % HB;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float prev = (hb == 0 && i == 0) ? 0.f : s[kb];
                s[kb] = fmaf(w[hb][i], RELU ? relu(x[i]) : x[i], prev);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Reduce-scatter over the four 16-lane groups: lane g*16+c returns
// sum over groups of s[g] at column c, i.e. the full head sum of key g*16+c.
// permlane32_swap(x, y) exchanges the upper half of x with the lower half of
// y; adding both results folds the two halves.  permlane16_swap does the same
// between 16-lane rows 0/1 and 2/3.
__device__ __forceinline__ float reduce_scatter4(const float (&s)[4]) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(s[0]), __float_as_uint(s[2]), false, false);
    const float ta = __uint_as_float(p[0]) + __uint_as_float(p[1]);  // rows 0,1: sum s0; rows 2,3: sum s2
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(s[1]), __float_as_uint(s[3]), false, false);
    const float tb = __uint_as_float(q[0]) + __uint_as_float(q[1]);  // rows 0,1: sum s1; rows 2,3: sum s3
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(ta), __float_as_uint(tb), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Pool page of block blk of a row's table (-1: past the table or out of the
// pool).  The unchecked form requires max_blocks > 0.
__device__ __forceinline__ int32_t page_of_unchecked(const ScoreParams& p, int64_t row, int32_t blk) {
    const int32_t page = p.table[row * p.table_stride + min(max(blk, 0), p.max_blocks - 1)];
    return ((blk < p.max_blocks) & (page >= 0) & (page < p.kv_blocks)) ? page : -1;
}

__device__ __forceinline__ int32_t page_of(const ScoreParams& p, int64_t row, int32_t blk) {
    return p.max_blocks > 0 ? page_of_unchecked(p, row, blk) : -1;
}

__device__ __forceinline__ void store_logit(const ScoreParams& p, int64_t row, int32_t j, int32_t ctx, float v) {
    if (row >= p.rows || j >= p.max_context_len) return;
    if (j < ctx)
        p.logits[row * p.logits_stride + j] = v;
    else if (p.clean)
        p.logits[row * p.logits_stride + j] = -__builtin_huge_valf();
}

// ------------------------------------------------------------ shared table
// Key pages are moved HBM -> LDS by buffer loads with the LDS destination
// (one 16-byte chunk per lane, 1 KiB per wave instruction) into a ring of
// kStages page buffers.  A page's MFMA B fragments are read from LDS into
// registers one step before the page is computed, so its buffer is refilled
// kStages pages ahead.  In LDS a page keeps its 128-byte key rows but chunk c
// of key k sits in slot c ^ key_swizzle(k): any 8 (and any 16 aligned)
// consecutive keys of one chunk then hit distinct 16-byte bank groups, for
// both 128- and 256-byte bank rows.  Invalid pages use a buffer descriptor of
// zero length, which makes every load return zeros.
constexpr int kStages = 4;
constexpr int kDmaPerPage = 3;  // per wave: two 1 KiB key chunks + 64 bytes of scales

__device__ __forceinline__ int key_swizzle(int k) { return (k ^ (k >> 3)) & 7; }

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));


// Raw buffer descriptor over one native page.
__device__ __forceinline__ i32x4 page_rsrc(const uint8_t* kv, int32_t page) {
    const uint64_t base = reinterpret_cast<uint64_t>(kv + (int64_t)max(page, 0) * V1_PAGE_BYTES);
    return i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)(base >> 32) & 0xffff, page >= 0 ? V1_PAGE_BYTES : 0,
                 kRawDword};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((lds_ptr)(const_cast<void*>(p)));
}

// Buffer loads whose data goes to LDS at M0 + 16 (or 4) * lane.  Issued as
// inline assembly so that the compiler keeps no bookkeeping of its own for
// them: every wait on them is the explicit one before the page barrier.
// The descriptor and LDS address are wave-uniform; readfirstlane pins them
// to scalar registers.  No other code in these kernels uses M0.
__device__ __forceinline__ i32x4 uniform(const i32x4& v) {
    return i32x4{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                 __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
}
__device__ __forceinline__ void dma16(const i32x4& rs, int32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(voff), "s"(uniform(rs)), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const i32x4& rs, int32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
                 :: "v"(voff), "s"(uniform(rs)), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// Waits until this wave has at most `pending` page loads in flight (so the
// older page has landed), drains its LDS traffic, then joins the work-group
// barrier.  The memory clobber keeps the compiler from moving LDS accesses
// across it; no fence is used, as a fence would drain every load.
#define V1_PAGE_BARRIER(pending) \
    asm volatile("s_waitcnt vmcnt(" #pending ") lgkmcnt(0)\n\ts_barrier" ::: "memory")

// Work items are (8-query group, range of consecutive chunks of up to
// kMaxRangePages pages).  A persistent work-group pulls items from a counter,
// so work-groups that run faster (or drew shorter rows) take more of them and
// the kernel ends within about one item of the average.  An item walks its
// chunks through one continuous page ring, so the query fragments, weights
// and page ids are loaded once per item; each page's logits are stored from
// registers as soon as they are computed.
constexpr int kMaxRangePages = 256;
constexpr int kMarkWords = kMaxRangePages / 32 + 1;  // an item's pages start at a multiple of 16

// Union form (per-row tables): an item is a range of at most kUnionRange of a
// group's union entries (one per lane of a wave); items are listed per level,
// full ranges (level 0) before the halving tail (levels 1 ..).
constexpr int kUnionRange = 64;
constexpr int kUnionLevels = 10;
static_assert(kUnionRange == kWave && kUnionRange <= kMaxRangePages, "one union entry per lane");

// UNION: the item's pages are union entries of per-row tables (their columns
// come from each row's table slot; a wave skips the MFMAs of a page none of
// its queries lists, while the ring, the barriers and the store count go on
// unchanged).  QPW: queries per wave, 2 (4 waves per group of 8 queries) or,
// for the union form, 1 (8 waves of 512 threads, each skipping the pages its
// own query does not list; the linear-term row block then carries the one
// query's pieces in rows r with r % 4 < 2 and zeros elsewhere, so every value
// is the same as with two queries per wave).
template <int HB, bool RELU, bool UNION = false, int QPW = kQueriesPerWave>
__global__ __launch_bounds__(kWave * kQueriesPerGroup / QPW) void score_shared(ScoreParams p) {
    static_assert(QPW == 2 || (QPW == 1 && UNION), "one query per wave: the union form");
    // ReLU through the linear term + |x| fold (and score_exact for exact
    // zeros) from two head blocks on; with one head block each result is
    // taken as w * max(x, 0) directly (exactly 0 when no head dot is
    // positive): its VALU cost is that of the fold's, and it saves the
    // linear-term MFMA (a third of the block's) and the exact pass.  The
    // union form (per-row tables) takes ReLU directly at every head count:
    // its values are then those of score_rows and the page-major kernels,
    // bit for bit, whichever of them scores a row.
    constexpr bool kFold = RELU && HB > 1 && !UNION;
    constexpr int kWaves = kQueriesPerGroup / QPW;
    constexpr int kBlock = kWave * kWaves;
    constexpr int kKeyDma = 8 / kWaves;       // 1 KiB key chunks per wave and page
    constexpr int kScaleLanes = 64 / kWaves;  // lanes loading the page's 256 bytes of scales
    __shared__ __attribute__((aligned(16))) uint8_t st0[V1_PAGE_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t st1[V1_PAGE_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t st2[V1_PAGE_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t st3[V1_PAGE_BYTES];
    // One query per wave (one work-group per CU): a ring of two windows of
    // kWin pages and one barrier per window.  The waves skip different pages
    // (each its own row's), so a barrier per page would hold them all to the
    // busiest SIMD at every page; over a window the loads even out.
    constexpr int kWin = 8;
    __shared__ __attribute__((aligned(16))) uint8_t ring[QPW == 1 ? 2 * kWin : 1][V1_PAGE_BYTES];
    __shared__ int32_t pids[kMaxRangePages];
    __shared__ int32_t item_sh;
    // ReLU path: per query of the group, a bitmap of the item's pages that
    // hold a key marked for the exact form (bit (page_begin % 32) + page);
    // all zero between items.
    __shared__ uint32_t marks[kFold && !UNION ? kQueriesPerGroup * kMarkWords : 1];
    const int t = threadIdx.x, l = __lane_id(), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (kFold && !UNION)
        for (int i = t; i < kQueriesPerGroup * kMarkWords; i += kBlock) marks[i] = 0u;
    // union items per level (final before this kernel starts)
    int32_t lvl_n[UNION ? kUnionLevels : 1];
    int32_t total_items = p.items;
    if constexpr (UNION) {
        total_items = 0;
#pragma unroll
        for (int L = 0; L < kUnionLevels; ++L) {
            lvl_n[L] = __builtin_amdgcn_readfirstlane(p.u_level_n[L]);
            total_items += lvl_n[L];
        }
    }
  for (;;) {
    // every wave has finished the previous item (its LDS is free) when the
    // next one is drawn
    __syncthreads();
    if (t == 0) item_sh = (int32_t)atomicAdd(p.work, 1u);
    __syncthreads();
    const int32_t item = __builtin_amdgcn_readfirstlane(item_sh);
    if (item >= total_items) break;
    int32_t group, page_begin, nchunk = 0, ulen = 0;
    int64_t ubase = 0;  // union: the item's first entry
    if constexpr (UNION) {
        int32_t idx = item, L = 0;
#pragma unroll
        for (int k = 0; k < kUnionLevels - 1; ++k)
            if (L == k && idx >= lvl_n[k]) {
                idx -= lvl_n[k];
                L = k + 1;
            }
        const int2 it = reinterpret_cast<const int2*>(p.u_items)[(int64_t)L * p.u_level_stride + idx];
        group = __builtin_amdgcn_readfirstlane(it.x);
        page_begin = __builtin_amdgcn_readfirstlane(it.y) & 0xffff;
        ulen = __builtin_amdgcn_readfirstlane(it.y) >> 16;
        ubase = (int64_t)group * p.u_cap + page_begin;
    } else {
        group = item % p.groups;
        const int32_t level = item / p.groups;
        const int32_t c_begin = level < p.bulk ? level * p.full : p.lvl_start[level - p.bulk];
        nchunk = level < p.bulk ? p.full : p.lvl_chunks[level - p.bulk];
        page_begin = c_begin * kChunkPages;
    }
    const int64_t row0 = (int64_t)group * kQueriesPerGroup;
    const int32_t grows = (int32_t)min<int64_t>(kQueriesPerGroup, (int64_t)p.rows - row0);  // rows of the group

    // The independent loads of the prologue are all issued before the first
    // wait: query lengths (lane q mod 8: query row0 + q), the range's page
    // ids, query fragments, weights and records.
    int32_t lane_ctx;
    {
        const int64_t r = row0 + (l & (kQueriesPerGroup - 1));
        const int32_t c = min(p.ctx[min(r, (int64_t)p.rows - 1)], p.max_context_len);
        lane_ctx = r < p.rows ? c : 0;
    }
    int32_t pid[1];
    static_assert(kMaxRangePages == kThreads && (kBlock == kThreads || UNION), "one page id per thread");
    // Union: lane l of every wave holds entry l's table slots for the wave's
    // two queries, packed as 16-bit halves (0xffff: not listed; slots are
    // below kUnionEntries), loaded with the prologue.
    uint32_t uslots = 0xffffffffu;
    if constexpr (UNION) {
        pid[0] = p.u_pages[ubase + min(t, ulen - 1)];
        if (t >= ulen) pid[0] = -1;
    } else if (p.max_blocks > 0) {
#pragma unroll
        for (int k = 0; k < kMaxRangePages / kThreads; ++k) pid[k] = page_of_unchecked(p, row0, page_begin + k * kThreads + t);
    } else {
#pragma unroll
        for (int k = 0; k < kMaxRangePages / kThreads; ++k) pid[k] = -1;
    }
    uint64_t umark[QPW] = {};  // union: item pages holding keys for the exact form
    uint64_t use_mask = ~0ull;  // union: item pages one of this wave's queries lists
    // Query fragments, weights and linear-term coefficients.  Rows past the
    // end read the last row (their logits are never stored).
    v8i a[QPW][HB];
    float w[QPW][HB][4];
    // Linear-term MFMA row block: row r holds piece 2*(r/4) + r%2 of query
    // (r/2)%2, so result row 4*(l/16)+i of lane l is piece 2*(l/16) + i%2 of
    // query i/2, and coef[i] is that piece's scale.  (One query per wave:
    // rows with r % 4 >= 2 are zero.)
    float coef[2 * QPW];
    float exact_thr[QPW];
    v8i alin = v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
        const int64_t r = row0 + wv * QPW + q;
        load_q<HB>(p, r, a[q]);
        const uint8_t* rec = p.pieces + min(r, (int64_t)p.rows - 1) * kPieceRowBytes;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const v4f x = *reinterpret_cast<const v4f*>(rec + kRecWeights + (hb * 16 + 4 * (l >> 4)) * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) w[q][hb][i] = x[i];
        }
        if (kFold) {
            const float2 x = *reinterpret_cast<const float2*>(rec + kRecScales + 8 * (l >> 4));
            coef[2 * q] = x.x;
            coef[2 * q + 1] = x.y;
            exact_thr[q] = *reinterpret_cast<const float*>(rec + kRecBound);  // the same for every lane
        }
    }
    if (kFold) {
        const int rr = l & 15;
        const int64_t rq = min(row0 + wv * QPW + (QPW == 2 ? (rr >> 1) & 1 : 0), (int64_t)p.rows - 1);
        const int piece = 2 * (rr >> 2) + (rr & 1);
        const u32x4* src = reinterpret_cast<const u32x4*>(p.pieces + rq * kPieceRowBytes + piece * 128 + 32 * (l >> 4));
        const u32x4 x = src[0], y = src[1];
        alin = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
        if (QPW == 1 && (rr & 2)) alin = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    }
    if (kBlock == kMaxRangePages || t < kMaxRangePages) pids[t] = pid[0];

    int32_t ctx[QPW];
    int32_t max_ctx = 0;
#pragma unroll
    for (int q = 0; q < kQueriesPerGroup; ++q) max_ctx = max(max_ctx, __builtin_amdgcn_readlane(lane_ctx, q));
#pragma unroll
    for (int q = 0; q < QPW; ++q) ctx[q] = __builtin_amdgcn_readlane(lane_ctx, wv * QPW + q);
    // pages of the range below the group's longest context (union: every entry)
    const int32_t npages = UNION ? ulen : max(0, min(nchunk * kChunkPages, (max_ctx + 63) / 64 - page_begin));

    // Pages of the item past the group's longest context are computed by
    // nobody: with clean_logits their columns below max_context_len get -inf.
    // (Union: the plan fills the columns past each row's last page.)
    auto fill_rest = [&](int32_t from_page) __attribute__((always_inline)) {
        if (UNION || !p.clean) return;
        for (int32_t pg = from_page; pg < nchunk * kChunkPages; ++pg) {
#pragma unroll
            for (int q = 0; q < QPW; ++q)
                store_logit(p, row0 + wv * QPW + q, (page_begin + pg) * 64 + l, ctx[q], 0.f);
        }
    };
    if (npages == 0) {
        fill_rest(0);
        continue;
    }
    __syncthreads();  // page ids in LDS

    // per-lane load offsets (into the page) of this wave's loads
    int32_t voff[kKeyDma];
#pragma unroll
    for (int i = 0; i < kKeyDma; ++i) {
        const int s = (kKeyDma * wv + i) * 64 + l;  // 16-byte LDS slot
        const int key = s >> 3;
        voff[i] = key * 128 + (((s & 7) ^ key_swizzle(key & 15)) << 4);
    }
    const int32_t soff = 8192 + 4 * kScaleLanes * wv + 4 * l;
    auto issue = [&](uint8_t* buf, int32_t page) {
        const i32x4 rs = page_rsrc(p.kv, page);
        const uint32_t base = lds_addr(buf);
#pragma unroll
        for (int i = 0; i < kKeyDma; ++i) dma16(rs, voff[i], base + (kKeyDma * wv + i) * 1024);
        if (l < kScaleLanes) dma4(rs, soff, base + 8192 + 4 * kScaleLanes * wv);
    };
    int32_t pid_next = 0;
    if constexpr (QPW == 2) {
        issue(st0, __builtin_amdgcn_readfirstlane(pids[0]));
        issue(st1, 1 < npages ? __builtin_amdgcn_readfirstlane(pids[1]) : -1);
        issue(st2, 2 < npages ? __builtin_amdgcn_readfirstlane(pids[2]) : -1);
        issue(st3, 3 < npages ? __builtin_amdgcn_readfirstlane(pids[3]) : -1);
        // page id of the next page to load, read from LDS one step ahead
        pid_next = pids[kStages];
    } else {
        // the first two windows
#pragma unroll
        for (int j = 0; j < 2 * kWin; ++j)
            issue(ring[j], j < npages ? __builtin_amdgcn_readfirstlane(pids[j]) : -1);
    }

    // B fragment of key block kb: key kb*16 + l%16, chunks 2*(l/16) and +1;
    // plus the scale of key l
    const int swz = key_swizzle(l & 15);
    const int boff0 = (l & 15) * 128 + (((2 * (l >> 4)) ^ swz) << 4);
    const int boff1 = (l & 15) * 128 + (((2 * (l >> 4) + 1) ^ swz) << 4);
    struct Frag {
        v8i b[4];
        float scale;
    };
    auto load_frag = [&](const uint8_t* buf, Frag& f) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(buf + kb * 2048 + boff0);
            const u32x4 y = *reinterpret_cast<const u32x4*>(buf + kb * 2048 + boff1);
            f.b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
        }
        f.scale = reinterpret_cast<const float*>(buf + 8192)[l];
    };

    // A page is one stream of kTotal MFMAs: per key block the linear-term
    // block (ReLU form), then each query's head blocks.  Result idx is folded
    // into the per-lane partials kLag MFMAs after it is issued, so the MFMA
    // pipe keeps working while the VALU folds older results; the stream runs
    // on across pages, the first kLag slots of a page finishing the previous
    // page's partials.
    constexpr int kPer = (kFold ? 1 : 0) + QPW * HB;
    constexpr int kTotal = 4 * kPer;
    constexpr int kLag = 3;
    static_assert(kTotal % (kLag + 1) == 0 && kTotal > kLag + 4, "result ring continues across pages");
    // slots of the page-boundary work inside the stream: the previous page's
    // logits are stored once its partials are complete, then the page
    // barrier and the next load are issued, then the next page's fragments read
    constexpr int kStoreAt = kLag - 1, kSyncAt = kLag + 2, kFragAt = kLag + 4;
    v4f d[kLag + 1];
#pragma unroll
    for (int k = 0; k <= kLag; ++k) d[k] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mfma_at = [&](int idx, const Frag& f) __attribute__((always_inline)) {
        const int kb = idx / kPer, r = idx % kPer;
        const int rr = kFold ? max(r - 1, 0) : r;  // head block (r == 0 is the linear-term block)
        d[idx % (kLag + 1)] = (kFold && r == 0) ? mfma_fp8(alin, f.b[kb]) : mfma_fp8(a[rr / HB][rr % HB], f.b[kb]);
    };
    auto consume = [&](int jj, float (&part)[QPW][4]) __attribute__((always_inline)) {
        const int kb = jj / kPer, r = jj % kPer;
        const v4f x = d[jj % (kLag + 1)];
        if (kFold && r == 0) {
#pragma unroll
            for (int q = 0; q < QPW; ++q) part[q][kb] = fmaf(coef[2 * q + 1], x[2 * q + 1], coef[2 * q] * x[2 * q]);
        } else {
            const int rr = kFold ? r - 1 : r;
            const int q = rr / HB, hb = rr % HB;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float prev = (!kFold && hb == 0 && i == 0) ? 0.f : part[q][kb];
                part[q][kb] = fmaf(w[q][hb][i], kFold ? fabsf(x[i]) : RELU ? relu(x[i]) : x[i], prev);
            }
        }
    };
    // Every step issues exactly QPW logit stores, each through a
    // buffer descriptor over the columns of the page that the query writes:
    // lanes with nothing to write (no page, a row past the end, a column past
    // max_context_len, or past the context without clean_logits) lie past the
    // descriptor's length, so the hardware's range check drops their stores.
    // The count of vector memory operations per step is then fixed, which
    // the page wait relies on.
    // Keys whose fast ReLU value lies within the query's exact-path threshold
    // of zero only mark their page here (a bit per query and page in LDS, set
    // in a rarely taken scalar branch with no vector memory operation); the
    // item's end hands the marks to score_exact.
    auto store = [&](int32_t pg, bool live, const float (&part)[QPW][4], float scale) {
#pragma unroll
        for (int q = 0; q < QPW; ++q) {
            const float v = reduce_scatter4(part[q]);
            const int32_t qr = wv * QPW + q;  // row within the group
            // this page's first column in the query's row (union: from the
            // row's table slot; a page the row does not list stores nothing)
            int32_t col = (page_begin + pg) * 64;
            bool lq = live;
            if constexpr (UNION) {
                const uint32_t half = ((uint32_t)__builtin_amdgcn_readlane((int)uslots, max(pg, 0)) >> (16 * q)) & 0xffffu;
                col = (int32_t)half * 64;
                lq = live && half != 0xffffu;
            }
            // columns [col, col + 64) of the query: logits below its context,
            // -inf from there to max_context_len with clean_logits; the
            // descriptor covers the columns to write, lanes past it are dropped
            const int32_t valid = ctx[q] - col;
            const int32_t end = (p.clean ? p.max_context_len : ctx[q]) - col;
            const int32_t lim = (lq && qr < grows && end > 0) ? (end < 64 ? end : 64) : 0;
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(p.logits + (row0 + qr) * p.logits_stride + col, 0,
                                                              lim * 4, kRawDword);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l < valid ? v * scale : -__builtin_huge_valf()), rs,
                                                  l * 4, 0, 0);
            if (kFold) {
                // (ballots of the bare compares stay scalar masks; the
                // uniform conditions join on the scalar side)
                const uint64_t near = __builtin_amdgcn_ballot_w64(fabsf(v) <= exact_thr[q]) &
                                      __builtin_amdgcn_ballot_w64(l < valid);
                if (near != 0ull && lq && qr < grows) {
                    if constexpr (UNION) {
                        // (a scalar bit per item page; handed out at the item's end)
                        umark[q] |= 1ull << (pg & 63);
                    } else {
                        // (the empty asm keeps this block's address arithmetic
                        // from being hoisted out of the loop into live registers)
                        int32_t bit = (page_begin & 31) + pg;
                        asm volatile("" : "+s"(bit));
                        if (l == 0)
                            atomicOr(&marks[(wv * QPW + q) * kMarkWords + (bit >> 5)], 1u << (bit & 31));
                    }
                }
            }
        }
    };

    // The store of a step with nothing to store: a descriptor of length 0
    // drops it, and the step's count of memory operations stays fixed.
    auto no_store = [&]() __attribute__((always_inline)) {
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(p.logits, 0, 0, kRawDword);
        __builtin_amdgcn_raw_buffer_store_b32(0u, rs, l * 4, 0, 0);
    };

    // The page wait.  A wave's vector memory operations complete in issue
    // order (loads and stores alike share vmcnt and retire in order), and per
    // step a wave issues QPW stores and then kDmaPerPage loads (kKeyDma key
    // chunks and the scales).  At step i the loads of page i+1 were issued at
    // step i-3; after them came the stores and loads of steps i-2 and i-1 and
    // the stores of step i, so `vmcnt <= kWaitCount` holds only once page i+1
    // has landed.  (The first pages are covered by the full wait before the
    // loop.)
    constexpr int kDmaPerPage = kKeyDma + 1;
    constexpr int kWaitCount = (kDmaPerPage + QPW) * (kStages - 2) + QPW;
    static_assert(kStages == 4 && (QPW == 1 || kWaitCount == 12), "barrier wait count (per page: two queries per wave)");
    // After the barrier every wave has read page i out of LDS (its fragments
    // were read at step i-1), so its buffer receives page i+4.
    auto sync = [&](int32_t i, uint8_t* cur) __attribute__((always_inline)) {
        V1_PAGE_BARRIER(12);  // kWaitCount
        issue(cur, i + kStages < npages ? __builtin_amdgcn_readfirstlane(pid_next) : -1);
        pid_next = pids[min(i + kStages + 1, kMaxRangePages - 1)];
    };
    auto drain = [&](float (&part)[QPW][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = kTotal - kLag; j < kTotal; ++j) consume(j, part);
    };
    // Page j is computed: it lies in the item and (union) one of this wave's
    // queries lists it.  (With 64 heads and two queries per wave the branch
    // around the stream costs the register allocator ~30 VGPRs past the 256
    // of two waves per SIMD: 64 heads take one query per wave.)
    constexpr bool kSkip = UNION;
    auto used = [&](int32_t j) __attribute__((always_inline)) {
        return j >= 0 && j < npages && (!kSkip || ((use_mask >> (j & 63)) & 1ull) != 0);
    };
    // Step i: page i's fragments are in fc; fn holds page i-1's until page
    // i+1's are read into it.
    auto step = [&](int32_t i, uint8_t* cur, const uint8_t* next, const Frag& fc, Frag& fn,
                    float (&pc)[QPW][4], float (&pp)[QPW][4]) {
        if (used(i)) {
#pragma unroll
            for (int idx = 0; idx < kTotal; ++idx) {
                mfma_at(idx, fc);
                // keep this order: the compiler would otherwise move each
                // consumer next to its MFMA and pad the gap with nops
                __builtin_amdgcn_sched_barrier(0);
                if (idx >= kLag)
                    consume(idx - kLag, pc);
                else
                    consume(kTotal + idx - kLag, pp);
                if (idx == kStoreAt) store(i - 1, used(i - 1), pp, fn.scale);
                if (idx == kSyncAt) sync(i, cur);
                if (idx == kFragAt) load_frag(next, fn);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // a page not computed (past the last page, or a union page this
            // wave's queries do not list): finish and store the previous
            // page if it was computed; the stores and loads of the step are
            // issued as in a computed one
            if (used(i - 1)) drain(pp);
            store(i - 1, used(i - 1), pp, fn.scale);
            sync(i, cur);
            load_frag(next, fn);
        }
    };
    // One query per wave, step i at position k of the ring: page i's
    // fragments are in fc (read during the previous step, or after the
    // barrier that opened its window); the previous page is stored (or, when
    // this wave did not compute it, a store through an empty descriptor is
    // issued, so every step issues exactly one); the next page's fragments
    // are read during the step unless it opens the next window.  At a
    // window's end the next window's loads were followed by exactly kWin
    // stores, every wave has read this window's pages, and its buffers
    // receive the window after next.
    // (ucur, uprev: this wave computes page i, computed page i - 1)
    auto wstep = [&](int32_t i, int k, bool ucur, bool uprev, const Frag& fc, Frag& fn, float (&pc)[QPW][4],
                     float (&pp)[QPW][4]) __attribute__((always_inline)) {
        const bool wend = k % kWin == kWin - 1;  // (k is a constant of the unrolled loop)
        uint8_t* next = ring[(k + 1) % (2 * kWin)];
        if (ucur) {
#pragma unroll
            for (int idx = 0; idx < kTotal; ++idx) {
                mfma_at(idx, fc);
                __builtin_amdgcn_sched_barrier(0);
                if (idx >= kLag)
                    consume(idx - kLag, pc);
                else
                    consume(kTotal + idx - kLag, pp);
                if (idx == kStoreAt) {
                    if (uprev)
                        store(i - 1, true, pp, fn.scale);
                    else
                        no_store();
                }
                if (idx == kFragAt && !wend) load_frag(next, fn);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            if (uprev) {
                drain(pp);
                store(i - 1, true, pp, fn.scale);
            } else {
                no_store();
            }
            if (!wend) load_frag(next, fn);
        }
        if (wend) {
            static_assert(kWin == 8, "window wait count");
            V1_PAGE_BARRIER(8);  // kWin
#pragma unroll
            for (int j = 0; j < kWin; ++j) {
                const int32_t pg = i + 1 + kWin + j;
                issue(ring[(k + 1 + kWin + j) % (2 * kWin)],
                      pg < npages ? __builtin_amdgcn_readfirstlane(pids[min(pg, kMaxRangePages - 1)]) : -1);
            }
            load_frag(next, fn);
        }
    };
    Frag fa, fb;
    float pa[QPW][4], pb[QPW][4];
#pragma unroll
    for (int q = 0; q < QPW; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) pa[q][k] = pb[q][k] = 0.f;
    // Compiler-visible full wait: the query fragments, weights and records
    // loaded above are complete before the loop, so no wait for them is
    // placed inside it.  (It also covers the first pages.)
    __builtin_amdgcn_s_waitcnt(0);
    V1_PAGE_BARRIER(0);
#pragma unroll
    for (int q = 0; q < QPW; ++q)
        exact_thr[q] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, exact_thr[q])));
    if constexpr (UNION) {
        // (loaded after the prologue's wait: kept out of its register peak)
        const int64_t e = ubase + min(l, ulen - 1);
        const uint32_t umask = p.u_mask[e];
        if constexpr (QPW == 2) {
            const int2 uslot2 = *reinterpret_cast<const int2*>(p.u_slots + e * kQueriesPerGroup + wv * QPW);
            const bool in0 = l < ulen && ((umask >> (wv * QPW)) & 1u);
            const bool in1 = l < ulen && ((umask >> (wv * QPW + 1)) & 1u);
            uslots = (in0 ? (uint32_t)uslot2.x & 0xffffu : 0xffffu) |
                     ((in1 ? (uint32_t)uslot2.y & 0xffffu : 0xffffu) << 16);
            use_mask = __builtin_amdgcn_ballot_w64(in0 | in1);
        } else {
            const int32_t uslot = p.u_slots[e * kQueriesPerGroup + wv];
            const bool in0 = l < ulen && ((umask >> wv) & 1u);
            uslots = (in0 ? (uint32_t)uslot & 0xffffu : 0xffffu) | 0xffff0000u;
            use_mask = __builtin_amdgcn_ballot_w64(in0);
        }
    }
    if constexpr (QPW == 2) {
        load_frag(st0, fa);
        for (int32_t i = 0; i < npages; i += kStages) {
            step(i, st0, st1, fa, fb, pa, pb);
            step(i + 1, st1, st2, fb, fa, pb, pa);
            step(i + 2, st2, st3, fa, fb, pa, pb);
            step(i + 3, st3, st0, fb, fa, pb, pa);
        }
        if (npages % kStages == 0 && used(npages - 1)) {
            drain(pb);
            store(npages - 1, true, pb, fb.scale);
        }
    } else {
        // this wave's pages of the item as one mask (npages <= 64), read
        // per step with constant shifts
        static_assert(kUnionRange == 64 && 64 % (2 * kWin) == 0, "item pages in one 64-bit mask");
        const uint64_t vmask = use_mask & (npages >= 64 ? ~0ull : (1ull << npages) - 1ull);
        bool uprev = false;
        load_frag(ring[0], fa);
        for (int32_t i0 = 0; i0 < npages; i0 += 2 * kWin) {
            const uint64_t wm = vmask >> i0;
#pragma unroll
            for (int k = 0; k < 2 * kWin; k += 2) {
                const bool u0 = (wm >> k) & 1ull, u1 = (wm >> (k + 1)) & 1ull;
                wstep(i0 + k, k, u0, uprev, fa, fb, pa, pb);
                wstep(i0 + k + 1, k + 1, u1, u0, fb, fa, pb, pa);
                uprev = u1;
            }
        }
        if (uprev) {  // (the item ended at a ring boundary on a computed page)
            drain(pb);
            store(npages - 1, true, pb, fb.scale);
        }
    }
    V1_PAGE_BARRIER(0);  // the page buffers are reused by the next item
    fill_rest(npages);
    if constexpr (UNION) {
        // marked pages to the rows' page bitmaps, at each row's table slot
        if (kFold) {
            const int32_t words = (((p.max_context_len + 63) >> 6) + 31) >> 5;
#pragma unroll
            for (int q = 0; q < QPW; ++q) {
                uint64_t m = umark[q];
                while (m != 0ull) {
                    const int32_t pg = __builtin_ctzll(m);
                    m &= m - 1;
                    const int32_t slot = (int32_t)(((uint32_t)__builtin_amdgcn_readlane((int)uslots, pg) >> (16 * q)) & 0xffffu);
                    if (l == 0)
                        atomicOr(p.exact_pages + (row0 + wv * QPW + q) * words + (slot >> 5), 1u << (slot & 31));
                }
            }
        }
        continue;
    }
    // Marked pages go to the per-row page bitmap that score_exact reads (an
    // OR per word that has a mark; the words are cleared for the next item).
    // (The bitmaps' row length follows from max_context_len.)
    int lane = l;
    asm volatile("" : "+v"(lane));  // keeps the lane arithmetic below inside the loop
    if (kFold && lane < QPW * kMarkWords) {
        const int q = lane / kMarkWords, k = lane % kMarkWords;
        const uint32_t bits = marks[(wv * QPW + q) * kMarkWords + k];
        if (bits != 0u) {
            const int32_t words = (((p.max_context_len + 63) >> 6) + 31) >> 5;
            atomicOr(p.exact_pages + (row0 + wv * QPW + q) * words + (page_begin >> 5) + k, bits);
            marks[(wv * QPW + q) * kMarkWords + k] = 0u;
        }
    }
  }
}

// ---------------------------------------------------------------- per row
// Work-group (x, row) takes the row's 16-page chunks x, x + gridDim.x, ...;
// wave wv takes pages wv, wv + 4, wv + 8, wv + 12 of each, so a wave's pages
// ascend.  The next page's key fragments and scale are loaded before the
// current page's MFMAs (one page load always in flight), and a work-group
// covers many pages so that work-group launches do not bound short rows.
// The work-group first resolves the pool pages of all its chunks into LDS
// (up to kRowPids), so a page's key loads never wait on its table entry.
constexpr int kRowPids = 2048;

template <int HB, bool RELU>
__global__ __launch_bounds__(kThreads) void score_rows(ScoreParams p) {
    __shared__ int32_t pid_s[kRowPids];
    const int l = __lane_id(), wv = threadIdx.x / kWave;
    const int64_t row = blockIdx.y;
    if (p.row_filter != nullptr && p.row_filter[row] == 0) return;
    const int32_t ctx = min(p.ctx[row], p.max_context_len);
    const int32_t row_pages = (ctx + 63) / 64;
    const int32_t all_pages = (p.max_context_len + 63) / 64;
    // page of step s of this wave (ascending in s); its slot in pid_s
    auto page_at = [&](int32_t s) __attribute__((always_inline)) {
        return (int32_t)(blockIdx.x + (s >> 2) * gridDim.x) * kChunkPages + wv + 4 * (s & 3);
    };
    const int32_t my_chunks = max(0, ((row_pages + kChunkPages - 1) / kChunkPages - (int32_t)blockIdx.x +
                                      (int32_t)gridDim.x - 1) / (int32_t)gridDim.x);
    const bool staged = my_chunks * kChunkPages <= kRowPids;
    if (staged) {
        for (int32_t li = threadIdx.x; li < my_chunks * kChunkPages; li += kThreads) {
            const int32_t pg = (int32_t)(blockIdx.x + (li / kChunkPages) * gridDim.x) * kChunkPages + li % kChunkPages;
            pid_s[li] = pg < row_pages ? page_of(p, row, pg) : -1;
        }
        __syncthreads();
    }
    auto pool_page = [&](int32_t s, int32_t pg) __attribute__((always_inline)) {
        return staged ? pid_s[(s >> 2) * kChunkPages + wv + 4 * (s & 3)] : page_of(p, row, pg);
    };
    int32_t s = 0;
    if (page_at(0) < row_pages) {
        v8i a[HB];
        float w[HB][4];
        load_q<HB>(p, row, a);
        load_w<HB>(p, row, w);
        auto fetch = [&](int32_t s, int32_t pg, v8i (&b)[4], float& scale) __attribute__((always_inline)) {
            const int32_t page = pool_page(s, pg);
            if (page < 0) return false;
            const uint8_t* base = p.kv + (int64_t)page * V1_PAGE_BYTES;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const u32x4* src = reinterpret_cast<const u32x4*>(base + (kb * 16 + (l & 15)) * 128 + 32 * (l >> 4));
                const u32x4 x = src[0], y = src[1];
                b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
            }
            scale = reinterpret_cast<const float*>(base + 8192)[l];
            return true;
        };
        auto compute = [&](int32_t pg, bool ok, const v8i (&b)[4], float scale) __attribute__((always_inline)) {
            float out = 0.f;
            if (ok) {
                float part[4];
                page_partials_lag<HB, RELU>(a, b, w, part);
                out = reduce_scatter4(part);
            } else {
                scale = 0.f;
            }
            store_logit(p, row, pg * 64 + l, ctx, out * scale);
        };
        v8i b0[4], b1[4];
        float s0 = 0.f, s1 = 0.f;
        bool ok0 = fetch(0, page_at(0), b0, s0), ok1 = false;
        for (;;) {
            const int32_t pg = page_at(s), nx = page_at(s + 1);
            if (nx < row_pages) ok1 = fetch(s + 1, nx, b1, s1);
            compute(pg, ok0, b0, s0);
            ++s;
            if (nx >= row_pages) break;
            const int32_t nx2 = page_at(s + 1);
            if (nx2 < row_pages) ok0 = fetch(s + 1, nx2, b0, s0);
            compute(nx, ok1, b1, s1);
            ++s;
            if (nx2 >= row_pages) break;
        }
    }
    // pages past the row's context: -inf (clean) up to max_context_len
    if (p.clean)
        for (int32_t pg = page_at(s); pg < all_pages; pg = page_at(++s)) store_logit(p, row, pg * 64 + l, ctx, 0.f);
}

// The marked pages of the shared-table ReLU kernel (one wave per row): each
// page's 64 keys recomputed the direct way, sum_h w_h * max(x_h, 0) as in
// score_rows, replacing the fast values (the stream order after score_shared
// makes these stores the last ones).  A page past the table or out of the pool
// scored exactly 0 already and is skipped.
template <int HB>
__global__ __launch_bounds__(256) void score_exact(ScoreParams p) {
    const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    const int l = __lane_id();
    if (row >= p.rows) return;
    const int32_t ctx = min(p.ctx[row], p.max_context_len);
    bool loaded = false;
    v8i a[HB];
    float w[HB][4];
    for (int32_t w0 = 0; w0 < p.exact_words; w0 += kWave) {
        const uint32_t mine = w0 + l < p.exact_words ? p.exact_pages[row * p.exact_words + w0 + l] : 0u;
        uint64_t words = __builtin_amdgcn_ballot_w64(mine != 0u);
        while (words) {
            const int src = __builtin_ctzll(words);
            words &= words - 1;
            uint32_t bits = (uint32_t)__builtin_amdgcn_readlane((int)mine, src);
            if (!loaded) {
                load_q<HB>(p, row, a);
                load_w<HB>(p, row, w);
                loaded = true;
            }
            while (bits) {
                const int32_t pg = (w0 + src) * 32 + __builtin_ctz(bits);
                bits &= bits - 1;
                const int32_t page = __builtin_amdgcn_readfirstlane(page_of(p, row, pg));
                if (page < 0) continue;
                const uint8_t* kp = p.kv + (int64_t)page * V1_PAGE_BYTES;
                v8i b[4];
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const u32x4* src4 = reinterpret_cast<const u32x4*>(kp + (kb * 16 + (l & 15)) * 128 + 32 * (l >> 4));
                    const u32x4 x = src4[0], y = src4[1];
                    b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
                }
                const float scale = reinterpret_cast<const float*>(kp + 8192)[l];
                float part[4];
                page_partials<HB, true>(a, b, w, part);
                // the lane exchanges of the fold need every lane: only the
                // store is predicated
                const float v = reduce_scatter4(part) * scale;
                const int32_t j = pg * 64 + l;
                if (j < ctx) p.logits[row * p.logits_stride + j] = v;
            }
        }
    }
}


// ---------------------------------------------------------- union plan
// Per-row tables of a batch whose rows share most of their pages (the rows
// of one prefill chunk) go through the shared-table kernel's page ring.  Per
// group of 8 rows, the valid pages of the rows' live table slots go into a
// hash set in LDS (open addressing, linear probing); every distinct page
// becomes a union entry holding the pool page, a mask of the rows that list
// it and each such row's slot.  A row that lists a page again puts that slot
// in an entry of its own.  Slots past the table or out of the pool get no
// entry: their columns are written here, 0 below the row's context and -inf
// from there to max_context_len with clean_logits (the values of a page of
// zeros in score_rows).  Entries follow the order of the hash slots, which
// depends on the order of insertion; no value depends on it.  The group's
// entries are cut into items of at most kUnionRange entries, full ranges
// first (level 0), then a halving tail (levels 1 ..), appended to per-level
// lists.  Groups whose rows share too little (fewer than two listed pairs
// per entry on average), or where a page probes more than kPlanProbes
// slots, are flagged for score_rows, whose values are the same bit for bit.
// One work-group per group; with clean_logits it also fills the columns past
// each row's last page.
constexpr int kUnionEntries = 8192;  // (row, slot) pairs of a group: 8 rows x 1024 table pages
static_assert(kUnionEntries < 0xffff, "union slots fit 16 bits");
constexpr int kPlanThreads = 512;
constexpr int kPlanPairs = kUnionEntries / kPlanThreads;  // pairs per thread
constexpr int kPlanProbes = 64;
// Hash slots per group: the smallest power of two, at least one per thread,
// that holds every pair of a group (load <= 1/2 wherever the group is shared);
// 8 bytes of dynamic LDS each.
inline int32_t plan_slots(int32_t max_pairs) {
    int32_t n = kPlanThreads;
    while (n < max_pairs) n <<= 1;
    return n;
}
constexpr int kUnionMinRows = 513;   // decode batches (the reference's <= 512 rows) keep score_rows

struct UnionOut {
    int32_t* pages;
    uint32_t* mask;
    int32_t* slots;
    int32_t* items;     // int2 per item
    int32_t* level_n;
    int32_t* fallback;  // [rows] 1: the row is scored by score_rows
};

// Exclusive prefix sum of one value per thread over the work-group; `total`
// is the sum of all.
__device__ __forceinline__ int32_t plan_scan(int32_t v, int32_t* part, int32_t& total) {
    const int w = threadIdx.x / kWave, l = __lane_id();
    int32_t inc = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int32_t o = __shfl_up(inc, off, kWave);
        if (l >= off) inc += o;
    }
    if (l == kWave - 1) part[w] = inc;
    __syncthreads();
    int32_t before = 0;
    total = 0;
#pragma unroll
    for (int k = 0; k < kPlanThreads / kWave; ++k) {
        const int32_t x = part[k];
        if (k < w) before += x;
        total += x;
    }
    __syncthreads();  // part is free again
    return before + inc - v;
}

// Dynamic LDS: hslots page keys (-1: empty) and hslots row masks (after the
// count, the slot's entry).
__global__ __launch_bounds__(kPlanThreads) void score_union_plan(ScoreParams p, UnionOut u, int32_t hslots) {
    extern __shared__ __attribute__((aligned(16))) int32_t plan_lds[];
    int32_t* hkey = plan_lds;
    uint32_t* hbits = reinterpret_cast<uint32_t*>(plan_lds + hslots);
    __shared__ int32_t part[kPlanThreads / kWave];
    __shared__ int32_t overflow;
    __shared__ int32_t by_mask[256];
    const int t = threadIdx.x, l = __lane_id(), wv = threadIdx.x / kWave;
    const int32_t g = blockIdx.x;
    const int64_t row0 = (int64_t)g * kQueriesPerGroup;
    const int32_t grows = (int32_t)min<int64_t>(kQueriesPerGroup, (int64_t)p.rows - row0);
    const int64_t gbase = (int64_t)g * p.u_cap;
    // live table slots per row and their offsets in the pair list
    int32_t off[kQueriesPerGroup + 1];
    off[0] = 0;
#pragma unroll
    for (int q = 0; q < kQueriesPerGroup; ++q) {
        const int32_t c = q < grows ? min(p.ctx[row0 + q], p.max_context_len) : 0;
        off[q + 1] = off[q] + (max(c, 0) + 63) / 64;
    }
    const int32_t E = off[kQueriesPerGroup];  // <= hslots
    auto row_of = [&](int32_t e) __attribute__((always_inline)) {
        int q = 0;
#pragma unroll
        for (int j = 1; j < kQueriesPerGroup; ++j) q += e >= off[j] ? 1 : 0;
        return q;
    };
    for (int32_t h = t; h < hslots; h += kPlanThreads) {
        hkey[h] = -1;
        hbits[h] = 0u;
    }
    if (t == 0) overflow = 0;
    __syncthreads();
    // pair e = t + k * kPlanThreads: res[k] = its hash slot (plus 0x10000 when
    // its row listed the page at another slot first), -1 for a slot without
    // a valid page, -2 past the pairs
    const int shift = 32 - __builtin_ctz((uint32_t)hslots);
    int32_t res[kPlanPairs];
    int32_t nvalid = 0, nrep = 0;
#pragma unroll
    for (int k = 0; k < kPlanPairs; ++k) {
        const int32_t e = t + k * kPlanThreads;
        res[k] = -2;
        if (e < E) {
            const int q = row_of(e);
            const int32_t page = page_of(p, row0 + q, e - off[q]);
            res[k] = -1;
            if (page >= 0) {
                ++nvalid;
                uint32_t h = ((uint32_t)page * 0x9e3779b1u) >> shift;
                int32_t found = -1;
                for (int i = 0; i < kPlanProbes; ++i) {
                    const int32_t old = atomicCAS(&hkey[h], -1, page);
                    if (old == -1 || old == page) {
                        found = (int32_t)h;
                        break;
                    }
                    h = (h + 1) & (uint32_t)(hslots - 1);
                }
                if (found < 0) {
                    atomicOr(&overflow, 1);
                } else {
                    const uint32_t rep = (atomicOr(&hbits[found], 1u << q) >> q) & 1u;
                    nrep += (int32_t)rep;
                    res[k] = found | (int32_t)(rep << 16);
                }
            }
        }
    }
    __syncthreads();
    // thread t's run of hash slots: [t * per, (t + 1) * per)
    const int32_t per = hslots / kPlanThreads;
    int32_t occ = 0;
    for (int32_t h = t * per; h < (t + 1) * per; ++h) occ += hkey[h] != -1 ? 1 : 0;
    int32_t Umain, D, V;
    plan_scan(occ, part, Umain);
    const int32_t first_rep = Umain + plan_scan(nrep, part, D);
    plan_scan(nvalid, part, V);
    const int32_t U = Umain + D;
    const bool shared = overflow == 0 && 2 * U <= V;
    // Entries of distinct pages, counted by their mask of rows, then dealt
    // so that every 8 consecutive entries take a like share of each mask:
    // the one-row-per-wave union form computes a window of 8 entries per
    // barrier, each wave its own row's, and the busiest SIMD sets the
    // window's time.  Rank r < 8W (W = Umain / 8 windows) goes to
    // (r % W) * 8 + r / W, the rest stay in place.
    for (int i = t; i < 256; i += kPlanThreads) by_mask[i] = 0;
    __syncthreads();
    int32_t rk[kPlanPairs];
#pragma unroll
    for (int i = 0; i < kPlanPairs; ++i) {
        const int32_t h = t * per + i;
        rk[i] = 0;
        if (i < per && hkey[h] != -1) rk[i] = atomicAdd(&by_mask[hbits[h] & 0xffu], 1);
    }
    __syncthreads();
    int32_t counted;
    const int32_t mask_start = plan_scan(t < 256 ? by_mask[t] : 0, part, counted);
    if (t < 256) by_mask[t] = mask_start;
    __syncthreads();
    if (shared) {
        const int32_t W = Umain / 8;
#pragma unroll
        for (int i = 0; i < kPlanPairs; ++i) {
            const int32_t h = t * per + i;
            if (i >= per || hkey[h] == -1) continue;
            const uint32_t m = hbits[h];
            const int32_t r = by_mask[m & 0xffu] + rk[i];
            const int32_t e = r < 8 * W ? (r % W) * 8 + r / W : r;
            u.pages[gbase + e] = hkey[h];
            u.mask[gbase + e] = m;
            hbits[h] = (uint32_t)e;
        }
    }
    __syncthreads();
    if (shared) {
        int32_t r = first_rep;
#pragma unroll
        for (int k = 0; k < kPlanPairs; ++k) {
            if (res[k] < 0) continue;
            const int32_t e = t + k * kPlanThreads;
            const int q = row_of(e);
            const int32_t slot = e - off[q], h = res[k] & 0xffff;
            int32_t ent = (int32_t)hbits[h];
            if (res[k] >> 16) {
                ent = r++;
                u.pages[gbase + ent] = hkey[h];
                u.mask[gbase + ent] = 1u << q;
            }
            u.slots[(gbase + ent) * kQueriesPerGroup + q] = slot;
        }
        // slots without a valid page: the whole wave writes each one's 64 columns
#pragma unroll
        for (int k = 0; k < kPlanPairs; ++k) {
            uint64_t inv = __builtin_amdgcn_ballot_w64(res[k] == -1);
            while (inv != 0ull) {
                const int32_t lane = __builtin_ctzll(inv);
                inv &= inv - 1;
                const int32_t e = wv * kWave + lane + k * kPlanThreads;
                const int q = row_of(e);
                const int32_t c = min(p.ctx[row0 + q], p.max_context_len);
                const int32_t j = (e - off[q]) * 64 + l;
                float* rp = p.logits + (row0 + q) * p.logits_stride;
                if (j < c)
                    rp[j] = 0.f;
                else if (p.clean && j < p.max_context_len)
                    rp[j] = -__builtin_huge_valf();
            }
        }
    }
    if (t < grows) u.fallback[row0 + t] = shared ? 0 : 1;
    if (shared && p.clean) {
        // columns past each row's last live page (score_rows fills them for flagged rows)
        for (int q = 0; q < grows; ++q) {
            float* rp = p.logits + (row0 + q) * p.logits_stride;
            for (int32_t j = (off[q + 1] - off[q]) * 64 + t; j < p.max_context_len; j += kPlanThreads)
                rp[j] = -__builtin_huge_valf();
        }
    }
    if (shared && t < kUnionLevels) {
        // thread 0: the full ranges (level 0); thread L >= 1: the L-th range
        // of the halving tail, if the group's entries reach it
        const int32_t bulk = U > 2 * kUnionRange ? (U - kUnionRange) / kUnionRange : 0;
        int32_t first = 0, count = 0, start = 0, len = 0;
        if (t == 0) {
            count = bulk;
        } else {
            int32_t e = bulk * kUnionRange;
            for (int L = 1; L <= t && e < U; ++L) {
                const int32_t left = U - e;
                const int32_t size = min(left == 1 ? 1 : (left + 1) / 2, kUnionRange);
                if (L == t) {
                    start = e;
                    len = size;
                    count = 1;
                }
                e += size;
            }
        }
        if (count > 0) first = atomicAdd(u.level_n + t, count);
        int32_t* it = u.items + 2 * ((int64_t)t * p.u_level_stride + first);
        if (t == 0) {
            for (int32_t b = 0; b < bulk; ++b) {
                it[2 * b] = g;
                it[2 * b + 1] = (b * kUnionRange) | (kUnionRange << 16);
            }
        } else if (count > 0) {
            it[0] = g;
            it[1] = start | (len << 16);
        }
    }
}

// ------------------------------------------- page-major per-row tables
// Per-row tables of a large batch over a small pool (a prefill chunk's fine
// tables over one request's pages).  A work item is (chunk c of kPmPages
// consecutive pool pages, block of kPmRows rows): it stages the chunk's pages
// in LDS once and computes every (row, listed page) pair of its rows from
// them, so every MFMA serves a row that lists the page and a key page is read
// from memory once per row block rather than once per row.  ReLU is taken
// directly (w * max(x, 0), as score_rows does), so a key with no positive
// head dot scores exactly 0 and no exact pass follows.
//   score_pages_clear  empties the dense pair table and the overflow count;
//   score_pages_place  one thread per (row, table slot): a listed pool page's
//                      slot goes to table[chunk][row][page % kPmPages]; a
//                      second slot of the same row and page goes to the
//                      overflow list; columns no pair covers are written
//                      (0 below the context: a slot past the table or out of
//                      the pool reads as zeros; -inf past it with clean_logits);
//   score_pages        the work items, plus one extra grid row that scores the
//                      overflow pairs one wave per pair.
constexpr int kPmPages = 8;
constexpr int kPmWaves = 4;                // waves per work-group
constexpr bool kPmPrefetch = true;         // the next row's loads issued before the current row
constexpr int kPmRows = 16 * kPmWaves;     // rows per work item
constexpr uint32_t kPmNone = 0xffffffffu;
constexpr int64_t kPmMaxTableBytes = 64ll << 20;

// Chunks are cut from the pool pages the batch lists, in pool order (a
// bitmap of listed pages and each page's rank among them), so a chunk's
// pages are all live even where the listed pages are spread over a larger
// pool (a fine pool of 2048 page slots holding 1024 built pages).
constexpr int kPmMaxPool = 32768;          // pool pages (a 1024-word bitmap)
constexpr int kPmReplicas = 16;            // copies of the bitmap the marks are spread over
constexpr int kPmMarkRows = 4;             // rows per work-group of the marks
constexpr int kPmRankThreads = 1024;

struct PmTables {
    uint32_t* table;      // [chunks][rows][kPmPages] table slot of (row, listed page), kPmNone: not listed
    uint32_t* overflow;   // (row << 16 | slot) of the pairs the table has no room for
    uint32_t* count;      // [0] overflow entries, [1] listed pool pages
    uint32_t* bits;       // [kPmReplicas][words] pool pages some row lists (replica 0: all, after the ranks)
    uint32_t* word_base;  // [words] listed pages before each bitmap word
    int32_t* listed;      // listed pool pages in pool order (the rank's page)
    int64_t table_words;  // 16-byte words of the table
    int32_t chunks;
    int32_t words;
    int32_t compact;      // chunks of listed pages (else of consecutive pool pages)
};

struct PmLayout {
    int64_t count, overflow, bits, word_base, listed, table, total, table_words;
    int32_t chunks, words;
};
PmLayout pm_layout(int32_t rows, int32_t max_context_len, int64_t kv_blocks) {
    PmLayout L{};
    auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
    L.chunks = (int32_t)cdiv(kv_blocks, kPmPages);
    L.words = (int32_t)cdiv(kv_blocks, 32);
    L.count = 0;
    L.overflow = 256;
    L.bits = up(L.overflow + (int64_t)rows * cdiv(max_context_len, 64) * 4);
    L.word_base = up(L.bits + (int64_t)kPmReplicas * L.words * 4);
    L.listed = up(L.word_base + (int64_t)L.words * 4);
    L.table = up(L.listed + kv_blocks * 4);
    const int64_t table_bytes = (int64_t)L.chunks * rows * kPmPages * 4;
    L.table_words = table_bytes / 16;
    L.total = L.table + table_bytes;
    return L;
}

__global__ __launch_bounds__(256) void score_pages_clear(PmTables m) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint4* s = reinterpret_cast<uint4*>(m.table);
    for (int64_t k = i0; k < m.table_words; k += stride) s[k] = make_uint4(kPmNone, kPmNone, kPmNone, kPmNone);
    for (int64_t k = i0; k < (int64_t)kPmReplicas * m.words; k += stride) m.bits[k] = 0u;
    if (i0 < 2) m.count[i0] = 0u;
}

// The listed-page bitmap: each work-group ORs the valid pages of
// kPmMarkRows rows' tables into an LDS bitmap, then its non-zero words into
// replica b % 16 of
// the global bitmap (a small pool's few words would otherwise take a global
// atomic from every work-group on one address); the rank kernel ORs the
// replicas.
__global__ __launch_bounds__(256) void score_pages_mark(ScoreParams p, PmTables m) {
    __shared__ uint32_t lb[kPmMaxPool / 32];
    const int t = threadIdx.x;
    for (int k = t; k < m.words; k += 256) lb[k] = 0u;
    __syncthreads();
    for (int rr = 0; rr < kPmMarkRows; ++rr) {
        const int64_t row = (int64_t)blockIdx.x * kPmMarkRows + rr;
        if (row >= p.rows) break;
        const int32_t row_pages = (min(p.ctx[row], p.max_context_len) + 63) / 64;
        for (int32_t j = t; j < row_pages; j += 256) {
            const int32_t page = page_of(p, row, j);
            if (page >= 0) atomicOr(&lb[page >> 5], 1u << (page & 31));
        }
    }
    __syncthreads();
    uint32_t* rep = m.bits + (int64_t)(blockIdx.x % kPmReplicas) * m.words;
    for (int k = t; k < m.words; k += 256)
        if (lb[k]) atomicOr(&rep[k], lb[k]);
}

// Ranks: one work-group, one bitmap word per thread (words <= 1024).
__global__ __launch_bounds__(kPmRankThreads) void score_pages_rank(PmTables m) {
    __shared__ uint32_t part[kPmRankThreads / kWave];
    const int t = threadIdx.x, w = t / kWave, l = __lane_id();
    uint32_t bits = 0u;
    if (t < m.words) {
#pragma unroll
        for (int r = 0; r < kPmReplicas; ++r) bits |= m.bits[(int64_t)r * m.words + t];
    }
    const uint32_t c = (uint32_t)__popc(bits);
    const uint32_t incl = wave_inclusive_sum(c);
    if (l == kWave - 1) part[w] = incl;
    __syncthreads();
    uint32_t base = incl - c;
    for (int k = 0; k < w; ++k) base += part[k];
    if (t < m.words) {
        m.word_base[t] = base;
        m.bits[t] = bits;  // (replica 0 becomes the union, which the place kernel reads)
    }
    uint32_t left = bits, at = base;
    while (left) {
        const int b = __builtin_ctz(left);
        left &= left - 1u;
        m.listed[at++] = t * 32 + b;
    }
    if (t == kPmRankThreads - 1) m.count[1] = base + c;
}

__global__ __launch_bounds__(256) void score_pages_place(ScoreParams p, PmTables m) {
    const int64_t row = blockIdx.y;
    const int32_t j = (int32_t)(blockIdx.x * 256 + threadIdx.x);
    const int32_t all_pages = (p.max_context_len + 63) / 64;
    if (j >= all_pages) return;
    const int32_t ctx = min(p.ctx[row], p.max_context_len);
    const int32_t row_pages = (ctx + 63) / 64;
    const int32_t page = j < row_pages ? page_of(p, row, j) : -1;
    if (page >= 0) {
        const uint32_t rank =
            m.compact ? m.word_base[page >> 5] + (uint32_t)__popc(m.bits[page >> 5] & ((1u << (page & 31)) - 1u))
                      : (uint32_t)page;
        uint32_t* at = m.table + (((int64_t)(rank / kPmPages) * p.rows + row) * kPmPages + rank % kPmPages);
        if (atomicCAS(at, kPmNone, (uint32_t)j) != kPmNone) m.overflow[atomicAdd(m.count, 1u)] = (uint32_t)(row << 16) | (uint32_t)j;
        return;
    }
    if (j >= row_pages && !p.clean) return;
    for (int i = 0; i < 64; ++i) store_logit(p, row, j * 64 + i, ctx, 0.f);
}

template <int HB, bool RELU>
__global__ __launch_bounds__(kWave * kPmWaves) void score_pages(ScoreParams p, PmTables m) {
    __shared__ __attribute__((aligned(16))) uint8_t pages[kPmPages][V1_PAGE_BYTES];
    __shared__ uint32_t used_sh;
    constexpr int kBlock = kWave * kPmWaves;
    const int t = threadIdx.x, l = __lane_id(), wv = __builtin_amdgcn_readfirstlane(t / kWave);
    // B fragment of key block kb of a staged page: key kb*16 + l%16, chunks
    // 2*(l/16) and +1 (stored swizzled, as score_shared stages them)
    const int swz = key_swizzle(l & 15);
    const int boff0 = (l & 15) * 128 + (((2 * (l >> 4)) ^ swz) << 4);
    const int boff1 = (l & 15) * 128 + (((2 * (l >> 4) + 1) ^ swz) << 4);
    if ((int32_t)blockIdx.y == m.chunks) {
        // overflow pairs: one wave per pair, the page read straight from memory
        const uint32_t n = *m.count;
        for (uint32_t e = blockIdx.x * kPmWaves + wv; e < n; e += gridDim.x * kPmWaves) {
            const uint32_t pr = m.overflow[e];
            const int64_t row = pr >> 16;
            const int32_t slot = (int32_t)(pr & 0xffffu);
            const int32_t page = page_of(p, row, slot);
            v8i a[HB], b[4];
            float w[HB][4];
            load_q<HB>(p, row, a);
            load_w<HB>(p, row, w);
            const uint8_t* base = p.kv + (int64_t)max(page, 0) * V1_PAGE_BYTES;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const u32x4* src = reinterpret_cast<const u32x4*>(base + (kb * 16 + (l & 15)) * 128 + 32 * (l >> 4));
                const u32x4 x = src[0], y = src[1];
                b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
            }
            const float scale = reinterpret_cast<const float*>(base + 8192)[l];
            float part[4];
            page_partials_lag<HB, RELU>(a, b, w, part);
            store_logit(p, row, slot * 64 + l, min(p.ctx[row], p.max_context_len), reduce_scatter4(part) * scale);
        }
        return;
    }
    const int32_t c = blockIdx.y;
    const int64_t r0 = (int64_t)blockIdx.x * kPmRows;
    const uint32_t* tab = m.table + (int64_t)c * p.rows * kPmPages;
    // pages of the chunk that the block's rows list
    if (t == 0) used_sh = 0;
    __syncthreads();
    uint32_t used = 0;
    for (int e = t; e < kPmRows * kPmPages; e += kBlock) {
        const int64_t r = r0 + e / kPmPages;
        if (r < p.rows && tab[r * kPmPages + e % kPmPages] != kPmNone) used |= 1u << (e % kPmPages);
    }
    if (used) atomicOr(&used_sh, used);
    __syncthreads();
    used = __builtin_amdgcn_readfirstlane(used_sh);
    if (used == 0) return;
    // stage the listed pages: per page eight 1 KiB key chunks and 256 bytes
    // of scales, the 72 loads dealt to the waves in turn
    const int32_t nlisted = m.compact ? __builtin_amdgcn_readfirstlane((int32_t)m.count[1]) : (int32_t)p.kv_blocks;
    for (int o = wv; o < kPmPages * 9; o += kPmWaves) {
        const int k = o / 9, part = o % 9;
        const int32_t idx = c * kPmPages + k;
        const int32_t page = !((used >> k) & 1u) || idx >= nlisted ? -1
                             : m.compact ? __builtin_amdgcn_readfirstlane(m.listed[min(idx, nlisted - 1)]) : idx;
        const i32x4 rs = page_rsrc(p.kv, page);
        const uint32_t base = lds_addr(pages[k]);
        if (part < 8) {
            const int s = part * 64 + l;  // 16-byte LDS slot
            const int key = s >> 3;
            dma16(rs, key * 128 + (((s & 7) ^ key_swizzle(key & 15)) << 4), base + part * 1024);
        } else {
            dma4(rs, 8192 + 4 * l, base + 8192);
        }
    }
    V1_PAGE_BARRIER(0);
    // Rows of this wave: r0 + wv, r0 + wv + 4, ...  The next row's table
    // slots, query fragments, weights and length are loaded before the
    // current row is computed (two register sets, used in turn); every load
    // is issued from a clamped index and every row issues exactly kPmPages
    // logit stores (range-checked buffer stores: a page the row does not list
    // gets a descriptor of length 0), so the wait for a row's data is an
    // exact count and never drains the next row's loads.
    const auto tab_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(tab), 0,
                                                          (int32_t)(p.rows * kPmPages * 4), kRawDword);
    const auto ctx_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(p.ctx), 0, p.rows * 4, kRawDword);
    const auto none_rs = __builtin_amdgcn_make_buffer_rsrc(p.logits, 0, 0, kRawDword);
    struct RowData {
        u32x4 s[kPmPages / 4];
        v8i a[HB];
        float w[HB][4];
        int32_t ctx;
    };
    // Whole head blocks (heads a multiple of 16): the query fragments and
    // weights load without the per-lane range selects (a row past the end
    // reads the last row, whose logits it never stores).
    const bool whole = (p.heads & 15) == 0;
    auto fetch = [&](int64_t row, RowData& d) __attribute__((always_inline)) {
        const int32_t rc = (int32_t)min(row, (int64_t)p.rows - 1);
#pragma unroll
        for (int i = 0; i < kPmPages / 4; ++i)
            d.s[i] = __builtin_amdgcn_raw_buffer_load_b128(tab_rs, rc * kPmPages * 4 + 16 * i, 0, 0);
        if (whole) {
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) {
                const int h = hb * 16 + (l & 15);
                const u32x4* src = reinterpret_cast<const u32x4*>(p.q + ((int64_t)rc * p.heads + h) * 128 + 32 * (l >> 4));
                const u32x4 x = src[0], y = src[1];
                d.a[hb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
                const v4f wv4 = *reinterpret_cast<const v4f*>(p.w + (int64_t)rc * p.heads + hb * 16 + 4 * (l >> 4));
#pragma unroll
                for (int i = 0; i < 4; ++i) d.w[hb][i] = wv4[i];
            }
        } else {
            load_q<HB>(p, row, d.a);
            load_w<HB>(p, row, d.w);
        }
        d.ctx = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(ctx_rs, rc * 4, 0, 0);
    };
    auto run = [&](int64_t row, const RowData& d) __attribute__((always_inline)) {
        uint32_t slot[kPmPages];
#pragma unroll
        for (int k = 0; k < kPmPages; ++k) slot[k] = d.s[k / 4][k % 4];
        const int32_t ctx = min(__builtin_amdgcn_readfirstlane(d.ctx), p.max_context_len);
        const bool live_row = row < p.rows;
#pragma unroll
        for (int k = 0; k < kPmPages; ++k) {
            const uint32_t sk = __builtin_amdgcn_readfirstlane(slot[k]);
            const bool live = live_row && sk != kPmNone;
            if (!live) {
                // (the store count stays fixed: a zero-length descriptor drops it)
                __builtin_amdgcn_raw_buffer_store_b32(0u, none_rs, 0, 0, 0);
                continue;
            }
            float v = 0.f;
            {
                v8i b[4];
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const u32x4 x = *reinterpret_cast<const u32x4*>(pages[k] + kb * 2048 + boff0);
                    const u32x4 y = *reinterpret_cast<const u32x4*>(pages[k] + kb * 2048 + boff1);
                    b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
                }
                float part[4];
                page_partials_lag<HB, RELU>(d.a, b, d.w, part);
                v = reduce_scatter4(part) * reinterpret_cast<const float*>(pages[k] + 8192)[l];
            }
            // columns [col, col + 64) of the row: logits below its context,
            // -inf from there to max_context_len with clean_logits
            const int32_t col = (int32_t)sk * 64;
            const int32_t end = (p.clean ? p.max_context_len : ctx) - col;
            const int32_t lim = __builtin_amdgcn_readfirstlane(end > 0 ? (end < 64 ? end : 64) : 0);
            // (the row's address made scalar explicitly: the descriptor must be)
            const uint64_t at = reinterpret_cast<uint64_t>(p.logits + min(row, (int64_t)p.rows - 1) * p.logits_stride + col);
            const uint64_t at_s = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(at >> 32)) << 32) |
                                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)at);
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<float*>(at_s), 0, lim * 4, kRawDword);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l < ctx - col ? v : -__builtin_huge_valf()), rs, l * 4,
                                                  0, 0);
        }
    };
    constexpr int kSteps = kPmRows / kPmWaves;
    static_assert(kSteps % 2 == 0, "rows taken in pairs");
    if constexpr (kPmPrefetch) {
        RowData d0, d1;
        fetch(r0 + wv, d0);
#pragma unroll 1
        for (int i = 0; i < kSteps; i += 2) {
            const int64_t ra = r0 + wv + kPmWaves * i;
            if (ra >= p.rows) break;
            fetch(ra + kPmWaves, d1);
            run(ra, d0);
            if (ra + kPmWaves >= p.rows) break;
            fetch(ra + 2 * kPmWaves, d0);
            run(ra + kPmWaves, d1);
        }
    } else {
#pragma unroll 1
        for (int i = 0; i < kSteps; ++i) {
            const int64_t ra = r0 + wv + kPmWaves * i;
            if (ra >= p.rows) break;
            RowData d0;
            fetch(ra, d0);
            run(ra, d0);
        }
    }
}

// -------------------------------------------- scoring without DeepGEMM
// The reference's Triton fallbacks for hosts without DeepGEMM or with the
// query optimisations off (runtime.py:450-466, 565-590).

// sglang/srt/layers/attention/v1_deepseek/kernels.py:475-486: page p of a row
// scores the max of its 8 center logits for p < max(n-1, 0) / 1024 * 16, else
// -inf.  One thread per (row, page).
__global__ __launch_bounds__(256) void reduce_centers_kernel(const float* logits, int64_t stride, const int32_t* lens,
                                                             float* scores, int32_t maxp) {
    const int64_t row = blockIdx.y;
    const int32_t pg = (int32_t)blockIdx.x * 256 + threadIdx.x;
    if (pg >= maxp) return;
    const int32_t pages = max(lens[row] - 1, 0) / 1024 * 16;
    float v = -__builtin_huge_valf();
    if (pg < pages) {
        const float* src = logits + row * stride + (int64_t)pg * 8;
#pragma unroll
        for (int g = 0; g < 8; ++g) v = fmaxf(v, src[g]);
    }
    scores[row * maxp + pg] = v;
}

// Center counts of the coarse scoring: 8 per built page, at most maxp pages.
__global__ __launch_bounds__(256) void center_lens_kernel(const int32_t* lens, int32_t* out, int32_t rows,
                                                          int32_t maxp) {
    const int32_t r = (int32_t)blockIdx.x * 256 + threadIdx.x;
    if (r < rows) out[r] = min(max(lens[r] - 1, 0) / 1024 * 16, maxp) * 8;
}

// kernels.py:248-320: the fine candidates of a row scored straight from the
// two pools.  Candidate i < take * 64 is slot i % 64 of fine page
// rt[selected[i / 64]], kept when its logical position members[page][slot]
// lies in [sink, tail) and below n; the next sink + n - tail candidates are
// the sink and tail tokens read from native pages through nt.  One wave per
// 64 candidates: the 16-key MFMA fragments of a fine block come from one page;
// a tail block's keys are located one by one.  Pages or ranks outside their
// tables, and candidates past count, score -inf.
struct FineExtra {
    const uint8_t* native;
    int64_t native_blocks;
    const int32_t* members;   // [fine pages, 64]
    const int32_t* rt;        // [rows, maxp]
    const int32_t* nt;        // [rows, np]
    const void* selected;     // [rows, take_stride], int32 or int64
    int32_t selected_bits;
    const int32_t* takes;
    int32_t maxp, np, take_stride, sink, window;
};

template <int HB, bool RELU>
__global__ __launch_bounds__(kThreads) void fine_scores(ScoreParams p, FineExtra f) {
    const int l = __lane_id(), wv = threadIdx.x / kWave;
    const int64_t row = blockIdx.y;
    const int32_t width = p.max_context_len;
    const int32_t block = (int32_t)blockIdx.x * 4 + wv;
    if (block * 64 >= width) return;
    const int32_t n = p.ctx[row], take = max(f.takes[row], 0);
    const int32_t sink = min(n, f.sink);
    const int32_t tail = max(sink, min(max(n - 1, 0) / 1024 * 1024, max(sink, n - f.window)));
    const int64_t count = (int64_t)take * 64 + sink + n - tail;
    const int32_t i = block * 64 + l;  // this lane's candidate
    float* out = p.logits + row * p.logits_stride;
    const float ninf = -__builtin_huge_valf();
    if ((int64_t)block * 64 >= count) {
        if (i < width) out[i] = ninf;
        return;
    }
    v8i b[4];
    float scale = 0.f;
    bool good;
    if (block < take) {
        int64_t rank = -1;
        if (block < f.take_stride)
            rank = f.selected_bits == 64 ? static_cast<const int64_t*>(f.selected)[row * f.take_stride + block]
                                         : static_cast<const int32_t*>(f.selected)[row * f.take_stride + block];
        const int32_t page = (rank >= 0 && rank < f.maxp) ? f.rt[row * f.maxp + rank] : -1;
        const bool ok = page >= 0 && page < p.kv_blocks;
        const uint8_t* base = p.kv + (int64_t)(ok ? page : 0) * V1_PAGE_BYTES;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            b[kb] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
            if (ok) {
                const u32x4* src = reinterpret_cast<const u32x4*>(base + (kb * 16 + (l & 15)) * 128 + 32 * (l >> 4));
                const u32x4 x = src[0], y = src[1];
                b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
            }
        }
        int32_t logical = -1;
        if (ok) {
            scale = reinterpret_cast<const float*>(base + 8192)[l];
            logical = f.members[(int64_t)page * 64 + l];
        }
        good = ok && logical >= sink && logical < tail && logical < n;
    } else {
        // candidate c of the sink/tail part: its native page and slot, or false
        auto locate = [&](int32_t c, int32_t& page, int32_t& logical) __attribute__((always_inline)) {
            if ((int64_t)c >= count) return false;
            const int32_t off = c - take * 64;
            logical = off < sink ? off : tail + off - sink;
            if (logical / 64 >= f.np) return false;
            page = f.nt[row * f.np + logical / 64];
            return page >= 0 && page < f.native_blocks;
        };
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            int32_t page = 0, logical = 0;
            b[kb] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
            if (locate(block * 64 + kb * 16 + (l & 15), page, logical)) {
                const u32x4* src = reinterpret_cast<const u32x4*>(f.native + (int64_t)page * V1_PAGE_BYTES +
                                                                  (logical % 64) * 128 + 32 * (l >> 4));
                const u32x4 x = src[0], y = src[1];
                b[kb] = v8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
            }
        }
        int32_t page = 0, logical = 0;
        good = locate(i, page, logical) && logical < n;
        if (good) scale = reinterpret_cast<const float*>(f.native + (int64_t)page * V1_PAGE_BYTES + 8192)[logical % 64];
    }
    v8i a[HB];
    float w[HB][4];
    load_q<HB>(p, row, a);
    load_w<HB>(p, row, w);
    float part[4];
    page_partials<HB, RELU>(a, b, w, part);
    const float v = reduce_scatter4(part) * scale;  // every lane takes part in the fold
    if (i < width) out[i] = good ? v : ninf;
}

struct Fine {
    template <int HB, bool RELU>
    static void launch(dim3 g, hipStream_t st, const ScoreParams& p, const FineExtra& f) {
        hipLaunchKernelGGL((fine_scores<HB, RELU>), g, dim3(kThreads), 0, st, p, f);
    }
};

struct Shared {
    template <int HB, bool RELU>
    static void launch(dim3 g, hipStream_t st, const ScoreParams& p) {
        hipLaunchKernelGGL((score_shared<HB, RELU>), g, dim3(kThreads), 0, st, p);
    }
};
// The union form (v1_score takes it from 17 heads): two queries per wave up
// to 48 heads, one with 64 (one 512-thread work-group per CU).
struct SharedUnion {
    template <int HB, bool RELU>
    static void launch(dim3 g, hipStream_t st, const ScoreParams& p) {
        if constexpr (HB == 2 || HB == 3)
            hipLaunchKernelGGL((score_shared<HB, RELU, true>), g, dim3(kThreads), 0, st, p);
        else if constexpr (HB == 4)
            hipLaunchKernelGGL((score_shared<HB, RELU, true, 1>), g, dim3(2 * kThreads), 0, st, p);
    }
};
struct Rows {
    template <int HB, bool RELU>
    static void launch(dim3 g, hipStream_t st, const ScoreParams& p) {
        hipLaunchKernelGGL((score_rows<HB, RELU>), g, dim3(kThreads), 0, st, p);
    }
};
struct Pages {
    template <int HB, bool RELU>
    static void launch(dim3 g, hipStream_t st, const ScoreParams& p, const PmTables& m) {
        hipLaunchKernelGGL((score_pages<HB, RELU>), g, dim3(kWave * kPmWaves), 0, st, p, m);
    }
};

template <typename K, int HB, typename... X>
void launch_relu(bool relu, dim3 g, hipStream_t st, const ScoreParams& p, const X&... x) {
    if (relu)
        K::template launch<HB, true>(g, st, p, x...);
    else
        K::template launch<HB, false>(g, st, p, x...);
}

template <typename K, typename... X>
void launch_hb(int hb, bool relu, dim3 g, hipStream_t st, const ScoreParams& p, const X&... x) {
    switch (hb) {
        case 1: launch_relu<K, 1>(relu, g, st, p, x...); break;
        case 2: launch_relu<K, 2>(relu, g, st, p, x...); break;
        case 3: launch_relu<K, 3>(relu, g, st, p, x...); break;
        default: launch_relu<K, 4>(relu, g, st, p, x...); break;
    }
}

}  // namespace
}  // namespace v1

using namespace v1;

// Shared-table workspace: per-query records, the work counter (256 bytes),
// then (ReLU rule) the per-row bitmaps of pages that score_exact recomputes.
static int32_t exact_words(int32_t max_context_len) { return (int32_t)cdiv(cdiv(max_context_len, 64), 32); }

extern "C" int64_t v1_score_workspace(int32_t rows, int32_t max_context_len) {
    if (rows <= 0 || max_context_len < 0) return 0;
    return (int64_t)rows * kPieceRowBytes + 256 + (int64_t)rows * exact_words(max_context_len) * 4;
}

// Per-row tables through the union plan: the shared-table workspace, then
// the plan (entries, masks, slots, items, level counts, row flags), each
// part 256-byte aligned.
namespace {
struct UnionLayout {
    int64_t pages, mask, slots, items, level_n, fallback, total;
    int32_t cap, level_stride;
};
static int64_t align_up(int64_t x) { return (x + 255) & ~int64_t(255); }
UnionLayout union_layout(int32_t rows, int32_t max_context_len) {
    UnionLayout L{};
    const int64_t groups = cdiv(rows, kQueriesPerGroup);
    L.cap = (int32_t)(kQueriesPerGroup * cdiv(max_context_len, 64));
    L.level_stride = (int32_t)(groups * (L.cap / kUnionRange + 2));
    int64_t at = align_up(v1_score_workspace(rows, max_context_len));
    L.pages = at;
    at = align_up(at + groups * L.cap * 4);
    L.mask = at;
    at = align_up(at + groups * L.cap * 4);
    L.slots = at;
    at = align_up(at + groups * L.cap * 4 * kQueriesPerGroup);
    L.items = at;
    at = align_up(at + (int64_t)kUnionLevels * L.level_stride * 8);
    L.level_n = at;
    at = align_up(at + kUnionLevels * 4);
    L.fallback = at;
    L.total = align_up(at + (int64_t)rows * 4);
    return L;
}
}  // namespace

extern "C" int64_t v1_score_tables_workspace(int32_t rows, int32_t max_context_len) {
    if (rows < kUnionMinRows || max_context_len <= 0 ||
        (int64_t)kQueriesPerGroup * cdiv(max_context_len, 64) > kUnionEntries)
        return 0;
    return union_layout(rows, max_context_len).total;
}

namespace {
int g_page_major = 1;
}

extern "C" int v1_score_page_major(int32_t enable, int32_t* previous) {
    V1_REQUIRE(enable == 0 || enable == 1, "score_page_major: enable must be 0 or 1 (got %d)", enable);
    if (previous) *previous = g_page_major;
    g_page_major = enable;
    return V1_OK;
}

extern "C" int64_t v1_score_pages_workspace(int32_t rows, int32_t max_context_len, int64_t kv_blocks) {
    // (overflow entries pack the row and the slot in 16 bits each)
    if (rows < kUnionMinRows || rows > 65535 || max_context_len <= 0 || cdiv(max_context_len, 64) > 65535 ||
        kv_blocks <= 0 || kv_blocks > kPmMaxPool)
        return 0;
    const PmLayout L = pm_layout(rows, max_context_len, kv_blocks);
    return L.total - L.table > kPmMaxTableBytes ? 0 : L.total;
}

extern "C" int v1_score(const v1_score_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "score: null args");
    V1_REQUIRE(a->heads >= 1 && a->heads <= 64, "score: heads must be in [1, 64]");
    V1_REQUIRE(a->rows >= 0 && a->max_context_len >= 0 && a->max_blocks >= 0, "score: bad shape");
    V1_REQUIRE(a->kv_blocks > 0, "score: empty key pool");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(a->q) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->kv_pages) & 15) == 0,
               "score: q and kv_pages must be 16-byte aligned");
    V1_REQUIRE(a->logits_stride >= a->max_context_len, "score: logits row stride too small");
    if (a->rows == 0 || a->max_context_len == 0) return V1_OK;
    ScoreParams p{a->q, a->kv_pages, a->kv_blocks, a->weights, a->context_lens, a->block_table, a->block_table_stride,
                  a->max_blocks, a->logits, a->logits_stride, a->max_context_len, a->rows, a->heads, a->relu,
                  a->clean_logits, nullptr};
    const int hb = (a->heads + 15) / 16;
    const uint32_t chunks = (uint32_t)cdiv(cdiv(a->max_context_len, 64), kChunkPages);
    hipStream_t st = as_stream(stream);
    if (a->block_table_stride == 0) {
        const int64_t need = v1_score_workspace(a->rows, a->max_context_len);
        V1_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need, "score: workspace of %lld bytes required",
                   (long long)need);
        V1_REQUIRE((reinterpret_cast<uintptr_t>(a->workspace) & 15) == 0, "score: workspace must be 16-byte aligned");
        // Work items: each row group's chunks cut into ranges that halve in
        // size (at most kMaxRangePages pages), all groups' largest ranges
        // first; work-groups pull them in that order, so the last ones taken
        // are short and the work-groups end together.  With few row groups
        // the full range shrinks so that the chunks make at least two items
        // per work-group: 1024 queries over 128 center pages (16 chunks of
        // max_context_len, 8 of them real) otherwise put each group's work in
        // one 128-page item on 128 of the 512 work-groups.
        const int64_t groups = cdiv(a->rows, kQueriesPerGroup);
        const int64_t wgs = 2 * (int64_t)v1::device_cus();
        const int64_t full = std::max<int64_t>(
            1, std::min<int64_t>(kMaxRangePages / kChunkPages, groups * (int64_t)chunks / (2 * wgs)));
        p.full = (int32_t)full;
        p.bulk = (int32_t)((int64_t)chunks > 2 * full ? ((int64_t)chunks - full) / full : 0);
        int nlevels = 0;
        for (int64_t c = (int64_t)p.bulk * full; c < (int64_t)chunks;) {
            const int64_t left = (int64_t)chunks - c;
            const int64_t size = std::min<int64_t>(left == 1 ? 1 : (left + 1) / 2, full);
            p.lvl_start[nlevels] = (int32_t)c;
            p.lvl_chunks[nlevels] = (int32_t)size;
            ++nlevels;
            c += size;
        }
        static_assert(kMaxLevels >= 8, "the halving tail of at most 2 full ranges has at most 7 levels");
        p.nchunks = (int32_t)chunks;
        p.groups = (int32_t)groups;
        const int64_t items = groups * ((int64_t)p.bulk + nlevels);
        V1_REQUIRE(items < (1ll << 31) - (1ll << 20), "score: too many work items");
        p.items = (int32_t)items;
        uint8_t* ws = static_cast<uint8_t*>(a->workspace);
        p.pieces = ws;
        p.work = reinterpret_cast<uint32_t*>(ws + (int64_t)a->rows * kPieceRowBytes);
        p.exact_pages = reinterpret_cast<uint32_t*>(ws + (int64_t)a->rows * kPieceRowBytes + 256);
        // ReLU: the linear term + |x| fold and score_exact from 17 heads on,
        // ReLU taken directly with one head block (score_shared's kFold)
        const bool fold = a->relu && hb > 1;
        p.exact_words = fold ? exact_words(a->max_context_len) : 0;
        const dim3 row_waves((uint32_t)cdiv(a->rows, 4));
        hipLaunchKernelGGL(score_prep, row_waves, dim3(256), 0, st, a->q, a->weights, a->rows, a->heads,
                           fold ? 1 : a->relu ? 2 : 0, ws, p.work, p.exact_pages, p.exact_words, nullptr, 0);
        int rc = V1_LAUNCHED("score_prep");
        if (rc != V1_OK) return rc;
        launch_hb<Shared>(hb, a->relu != 0, dim3((uint32_t)std::min<int64_t>(items, wgs)), st, p);
        rc = V1_LAUNCHED("score_shared");
        if (rc != V1_OK || !fold) return rc;
        switch (hb) {
            case 2: hipLaunchKernelGGL(score_exact<2>, row_waves, dim3(256), 0, st, p); break;
            case 3: hipLaunchKernelGGL(score_exact<3>, row_waves, dim3(256), 0, st, p); break;
            default: hipLaunchKernelGGL(score_exact<4>, row_waves, dim3(256), 0, st, p); break;
        }
        return V1_LAUNCHED("score_exact");
    }
    // Per-row tables of more than 512 rows and more than 16 heads over a pool
    // small enough for the dense pair table (one request's pages): the
    // page-major kernels.  Measured against the page-union plan: 4096 rows x
    // 32 heads (40 history pages + the shared tail union) 0.153 against
    // 0.182 ms; 1024 rows x 64 heads listing 545 of 1057 pages spread over a
    // 2116-page pool 0.424 against 0.463-0.48 ms (chunks of listed pages;
    // 0.493 ms in chunks of consecutive pool pages).  With one head block a
    // pair is 4 MFMAs and the placement kernels do not pay: 1024 rows x 16
    // heads of the reference example's fine tables 0.059 ms page-major
    // against 0.046 ms row by row.
    const int64_t pm_need = v1_score_pages_workspace(a->rows, a->max_context_len, a->kv_blocks);
    if (g_page_major && hb > 1 && pm_need > 0 && a->workspace != nullptr && a->workspace_bytes >= pm_need &&
        (reinterpret_cast<uintptr_t>(a->workspace) & 255) == 0) {
        const PmLayout L = pm_layout(a->rows, a->max_context_len, a->kv_blocks);
        uint8_t* ws = static_cast<uint8_t*>(a->workspace);
        const PmTables m{reinterpret_cast<uint32_t*>(ws + L.table), reinterpret_cast<uint32_t*>(ws + L.overflow),
                         reinterpret_cast<uint32_t*>(ws + L.count), reinterpret_cast<uint32_t*>(ws + L.bits),
                         reinterpret_cast<uint32_t*>(ws + L.word_base), reinterpret_cast<int32_t*>(ws + L.listed),
                         L.table_words, L.chunks, L.words,
                         // a pool more than twice a row's pages (listed pages spread thin)
                         a->kv_blocks > 2 * cdiv(a->max_context_len, 64)};
        const int64_t clear_wgs = std::max<int64_t>(1, std::min<int64_t>(cdiv(L.table_words, 256), 4 * (int64_t)v1::device_cus()));
        hipLaunchKernelGGL(score_pages_clear, dim3((uint32_t)clear_wgs), dim3(256), 0, st, m);
        int rc = V1_LAUNCHED("score_pages_clear");
        if (rc != V1_OK) return rc;
        if (m.compact) {
            hipLaunchKernelGGL(score_pages_mark, dim3((uint32_t)cdiv(a->rows, kPmMarkRows)), dim3(256), 0, st, p, m);
            rc = V1_LAUNCHED("score_pages_mark");
            if (rc != V1_OK) return rc;
            hipLaunchKernelGGL(score_pages_rank, dim3(1), dim3(kPmRankThreads), 0, st, m);
            rc = V1_LAUNCHED("score_pages_rank");
            if (rc != V1_OK) return rc;
        }
        hipLaunchKernelGGL(score_pages_place, dim3((uint32_t)cdiv(cdiv(a->max_context_len, 64), 256), (uint32_t)a->rows),
                           dim3(256), 0, st, p, m);
        rc = V1_LAUNCHED("score_pages_place");
        if (rc != V1_OK) return rc;
        launch_hb<Pages>(hb, a->relu != 0, dim3((uint32_t)cdiv(a->rows, kPmRows), (uint32_t)L.chunks + 1), st, p, m);
        return V1_LAUNCHED("score_pages");
    }
    // Per-row tables of more than 512 rows with a large enough workspace:
    // the union plan, the shared-table kernel over each group's union, and
    // score_rows for the rows of groups that share too little.
    // Measured: with one head block score_rows' cost per page (a few MFMAs)
    // is below the ring's; from 17 heads the waves skip the pages their rows
    // do not list (4096 rows x 32 heads, 40 routed pages: 0.31 -> 0.18 ms).
    const int64_t plan_need = v1_score_tables_workspace(a->rows, a->max_context_len);
    const bool plan = plan_need > 0 && a->heads > 16 && a->workspace != nullptr &&
                      a->workspace_bytes >= plan_need && (reinterpret_cast<uintptr_t>(a->workspace) & 255) == 0;
    if (plan) {
        const UnionLayout L = union_layout(a->rows, a->max_context_len);
        const int64_t groups = cdiv(a->rows, kQueriesPerGroup);
        uint8_t* ws = static_cast<uint8_t*>(a->workspace);
        p.pieces = ws;
        p.work = reinterpret_cast<uint32_t*>(ws + (int64_t)a->rows * kPieceRowBytes);
        p.exact_pages = reinterpret_cast<uint32_t*>(ws + (int64_t)a->rows * kPieceRowBytes + 256);
        p.exact_words = 0;  // (ReLU taken directly: no exact pass)
        p.groups = (int32_t)groups;
        p.u_cap = L.cap;
        p.u_level_stride = L.level_stride;
        UnionOut u{reinterpret_cast<int32_t*>(ws + L.pages), reinterpret_cast<uint32_t*>(ws + L.mask),
                   reinterpret_cast<int32_t*>(ws + L.slots), reinterpret_cast<int32_t*>(ws + L.items),
                   reinterpret_cast<int32_t*>(ws + L.level_n), reinterpret_cast<int32_t*>(ws + L.fallback)};
        p.u_pages = u.pages;
        p.u_mask = u.mask;
        p.u_slots = u.slots;
        p.u_items = u.items;
        p.u_level_n = u.level_n;
        const dim3 row_waves((uint32_t)cdiv(a->rows, 4));
        // (records of the weights alone: the union form takes ReLU directly)
        hipLaunchKernelGGL(score_prep, row_waves, dim3(256), 0, st, a->q, a->weights, a->rows, a->heads,
                           a->relu ? 2 : 0, ws, p.work, p.exact_pages, p.exact_words,
                           reinterpret_cast<uint32_t*>(u.level_n), (int32_t)kUnionLevels);
        int rc = V1_LAUNCHED("score_prep");
        if (rc != V1_OK) return rc;
        const int32_t hslots = plan_slots((int32_t)(kQueriesPerGroup * cdiv(a->max_context_len, 64)));
        // (dynamic LDS past 64 KiB needs the attribute, set once per process)
        static std::once_flag lds_once;
        static hipError_t lds_err = hipSuccess;
        std::call_once(lds_once, [] {
            lds_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&score_union_plan),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 8 * kUnionEntries);
        });
        if (lds_err != hipSuccess) return hip_status(lds_err, "score: hipFuncSetAttribute(score_union_plan)");
        hipLaunchKernelGGL(score_union_plan, dim3((uint32_t)groups), dim3(kPlanThreads), 8 * (size_t)hslots, st, p, u,
                           hslots);
        rc = V1_LAUNCHED("score_union_plan");
        if (rc != V1_OK) return rc;
        // (two 256-thread work-groups per CU; one of 512 threads with 64 heads)
        launch_hb<SharedUnion>(hb, a->relu != 0, dim3((uint32_t)((hb == 4 ? 1 : 2) * (int64_t)v1::device_cus())), st, p);
        rc = V1_LAUNCHED("score_shared (union)");
        if (rc != V1_OK) return rc;
        // flagged rows row by row (the same values, bit for bit), on score_rows' grid
        ScoreParams pr = p;
        pr.row_filter = u.fallback;
        int64_t per_row = std::max<int64_t>(1, std::min<int64_t>(chunks, cdiv(24 * (int64_t)v1::device_cus(), a->rows)));
        if (per_row > 1 && per_row % 2 == 0) --per_row;
        launch_hb<Rows>(hb, a->relu != 0, dim3((uint32_t)per_row, (uint32_t)a->rows), st, pr);
        return V1_LAUNCHED("score_rows (flagged rows)");
    }
    // About 24 work-groups per CU in all, each striding over its row's
    // chunks, and an odd count per row.  Work-groups are dealt to the 8 XCDs
    // in turn, so with a multiple of 8 per row one XCD takes the same chunk
    // positions of every row (on the 128-row decode batch 16 or 32 per row
    // ran 18-25% slower than 31, 33 or 47).
    int64_t per_row = std::max<int64_t>(1, std::min<int64_t>(chunks, cdiv(24 * (int64_t)v1::device_cus(), a->rows)));
    if (per_row > 1 && per_row % 2 == 0) --per_row;
    const dim3 grid((uint32_t)per_row, (uint32_t)a->rows);
    launch_hb<Rows>(hb, a->relu != 0, grid, st, p);
    return V1_LAUNCHED("score_rows");
}

// ---------------------------------------------- scoring without DeepGEMM
extern "C" int v1_reduce_centers(const float* logits, int64_t logits_stride, const int32_t* lens, float* scores,
                                 int32_t rows, int32_t maxp, void* stream) {
    V1_REQUIRE(rows >= 0 && maxp >= 0, "reduce_centers: negative shape");
    V1_REQUIRE(logits_stride >= 8ll * maxp, "reduce_centers: logits row stride below 8 * maxp");
    if (rows == 0 || maxp == 0) return V1_OK;
    hipLaunchKernelGGL(reduce_centers_kernel, dim3((uint32_t)cdiv(maxp, 256), (uint32_t)rows), dim3(256), 0,
                       as_stream(stream), logits, logits_stride, lens, scores, maxp);
    return V1_LAUNCHED("reduce_centers");
}

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

extern "C" int64_t v1_coarse_workspace(int32_t rows, int32_t maxp, int64_t table_stride) {
    if (rows <= 0 || maxp <= 0) return 0;
    return align256(4ll * rows) + align256(4ll * rows * 8 * maxp) +
           (table_stride == 0 ? v1_score_workspace(rows, 8 * maxp) : 0);
}

extern "C" int v1_coarse(const v1_coarse_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "coarse: null args");
    V1_REQUIRE(a->rows >= 0 && a->maxp >= 0 && a->maxp % 8 == 0, "coarse: maxp must be a non-negative multiple of 8");
    V1_REQUIRE(a->heads >= 1 && a->heads <= 64, "coarse: heads must be in [1, 64]");
    V1_REQUIRE(a->table_stride >= 0 && (a->table_stride == 0 || a->table_stride >= a->maxp / 8),
               "coarse: center table row stride below maxp / 8");
    if (a->rows == 0 || a->maxp == 0) return V1_OK;
    const int64_t need = v1_coarse_workspace(a->rows, a->maxp, a->table_stride);
    V1_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need, "coarse: workspace of %lld bytes required",
               (long long)need);
    V1_REQUIRE((reinterpret_cast<uintptr_t>(a->workspace) & 255) == 0, "coarse: workspace must be 256-byte aligned");
    uint8_t* ws = static_cast<uint8_t*>(a->workspace);
    int32_t* center_lens = reinterpret_cast<int32_t*>(ws);
    float* logits = reinterpret_cast<float*>(ws + align256(4ll * a->rows));
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(center_lens_kernel, dim3((uint32_t)cdiv(a->rows, 256)), dim3(256), 0, st, a->lens, center_lens,
                       a->rows, a->maxp);
    int rc = V1_LAUNCHED("coarse: center lengths");
    if (rc != V1_OK) return rc;
    // center logits of the built pages (columns past them -inf), then the max per page
    v1_score_args sa{};
    sa.q = a->q;
    sa.kv_pages = a->centers;
    sa.kv_blocks = a->center_blocks;
    sa.weights = a->weights;
    sa.context_lens = center_lens;
    sa.block_table = a->table;
    sa.block_table_stride = a->table_stride;
    sa.max_blocks = a->maxp / 8;
    sa.logits = logits;
    sa.logits_stride = 8ll * a->maxp;
    sa.max_context_len = 8 * a->maxp;
    sa.rows = a->rows;
    sa.heads = a->heads;
    sa.relu = a->relu;
    sa.clean_logits = 1;
    sa.workspace = ws + align256(4ll * a->rows) + align256(4ll * a->rows * 8 * a->maxp);
    sa.workspace_bytes = a->workspace_bytes - (align256(4ll * a->rows) + align256(4ll * a->rows * 8 * a->maxp));
    rc = v1_score(&sa, stream);
    if (rc != V1_OK) return rc;
    return v1_reduce_centers(logits, 8ll * a->maxp, a->lens, a->scores, a->rows, a->maxp, stream);
}

extern "C" int v1_fine(const v1_fine_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "fine: null args");
    V1_REQUIRE(a->heads >= 1 && a->heads <= 64, "fine: heads must be in [1, 64]");
    V1_REQUIRE(a->rows >= 0 && a->width >= 0 && a->maxp >= 0 && a->np >= 0 && a->take_stride >= 0,
               "fine: negative shape");
    V1_REQUIRE(a->selected_bits == 32 || a->selected_bits == 64, "fine: selected must be int32 or int64");
    V1_REQUIRE(a->fine_blocks > 0 && a->native_blocks > 0, "fine: empty pool");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(a->q) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->fine_pages) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a->native_pages) & 15) == 0,
               "fine: q and the pools must be 16-byte aligned");
    V1_REQUIRE(a->sink >= 0 && a->window >= 0, "fine: negative sink or window");
    if (a->rows == 0 || a->width == 0) return V1_OK;
    ScoreParams p{a->q, a->fine_pages, a->fine_blocks, a->weights, a->lens, nullptr, 0, 0, a->scores, a->width,
                  a->width, a->rows, a->heads, a->relu, 1, nullptr};
    FineExtra f{a->native_pages, a->native_blocks, a->members, a->rt, a->nt, a->selected, a->selected_bits, a->takes,
                a->maxp, a->np, a->take_stride, a->sink, a->window};
    const dim3 grid((uint32_t)cdiv(cdiv(a->width, 64), 4), (uint32_t)a->rows);
    launch_hb<Fine>((a->heads + 15) / 16, a->relu != 0, grid, as_stream(stream), p, f);
    return V1_LAUNCHED("fine");
}

// ------------------------------------------------ allocation-free variant
// The shared-table path's scratch (per-query records, work counter,
// exact-page bitmaps) in one static device array per GPU, for callers
// that cannot allocate.  Every call on a GPU shares that GPU's array: calls
// that overlap on one GPU race.  score_prep clears what must start at zero
// (the work counter and the bitmaps) with a kernel at every call.
constexpr int64_t kScratchBytes = 16ll << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// Device address of this GPU's scratch: hipGetSymbolAddress once per device,
// with that device current (the array's host-side name is not a device
// address and is never passed to a kernel).
int scratch_address(void* stream, void** out) {
    int cur = 0, dev = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_status(e, "score_noalloc: hipGetDevice");
    dev = cur;
    if (stream != nullptr) {
        e = hipStreamGetDevice(as_stream(stream), &dev);
        if (e != hipSuccess) return hip_status(e, "score_noalloc: hipStreamGetDevice");
    }
    V1_REQUIRE(dev >= 0 && dev < 64, "score_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return hip_status(e, "score_noalloc: hipSetDevice");
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess) return hip_status(e, "score_noalloc: hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return V1_OK;
}
}  // namespace

extern "C" int64_t v1_score_noalloc_capacity(void) { return kScratchBytes; }

extern "C" int v1_score_noalloc(const v1_score_args* a, void* stream) {
    V1_REQUIRE(a != nullptr, "score_noalloc: null args");
    v1_score_args b = *a;
    b.workspace = nullptr;
    b.workspace_bytes = 0;
    if (a->block_table_stride != 0) return v1_score(&b, stream);  // per-row tables use no scratch
    const int64_t need = v1_score_workspace(a->rows, a->max_context_len);
    V1_REQUIRE(need <= kScratchBytes,
               "score_noalloc: %d rows x %d columns need %lld bytes of scratch, more than the static %lld "
               "(call v1_score with a workspace)",
               a->rows, a->max_context_len, (long long)need, (long long)kScratchBytes);
    if (need > 0) {
        const int rc = scratch_address(stream, &b.workspace);
        if (rc != V1_OK) return rc;
        b.workspace_bytes = kScratchBytes;
    }
    return v1_score(&b, stream);
}
