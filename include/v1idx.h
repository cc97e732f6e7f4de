/*
 * v1idx.h -- C ABI of the MI355X (gfx950) query-indexing library `libv1idx.so`.
 *
 * Every entry point takes plain device pointers, element counts and strides,
 * and a HIP stream (passed as `void*`, i.e. a `hipStream_t`).  No entry point
 * allocates device memory, synchronises the stream or reads device data on the
 * host, so every launch is stream ordered and can be captured in a hipGraph.
 * Strides are in ELEMENTS of the pointed-to type unless the name ends in
 * `_bytes`.  FP8 data is OCP e4m3fn (`torch.float8_e4m3fn`), handled as bytes.
 *
 * Return value: V1_OK (0) or a negative V1_ERR_* code; `v1_last_error()` then
 * holds a message (thread local).  V1_ERR_INVALID means the arguments failed
 * validation and nothing was launched.
 *
 * A "native page" is 8448 bytes: 64 tokens x 128 FP8 bytes followed by 64 fp32
 * per-token scales (sglang/srt/layers/attention/v1_deepseek/kernels.py:1-3).
 */
#ifndef V1IDX_H
#define V1IDX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define V1_OK 0
#define V1_ERR_INVALID (-1)
#define V1_ERR_HIP (-2)
#define V1_ERR_UNSUPPORTED (-3)

#define V1_PAGE_TOKENS 64
#define V1_PAGE_BYTES 8448
#define V1_HEAD_DIM 128
#define V1_MAX_TOPK 2048
#define V1_TAIL_SCRATCH_PAGES 68

const char* v1_last_error(void);
int v1_abi_version(void);

/* ------------------------------------------------------------------------
 * fused.route: per-row page max-of-8, stable top-`take` page selection and
 * optional fine-page-table write.
 * Replaces V1QueryKernel::route
 *   sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:155-180 (kernel :7-49).
 * Ties between equal page maxima resolve to the lower page index.
 * ---------------------------------------------------------------------- */
typedef struct {
    const float* scores;      /* [batch, score_cols], row stride score_stride */
    int64_t score_stride;
    int32_t batch;
    int32_t score_cols;
    const int32_t* lens;      /* [batch] */
    const int32_t* takes;     /* [batch] */
    void* selected;           /* [batch, take_stride] int32 or int64 */
    int32_t selected_bits;    /* 32 or 64 */
    int32_t take_stride;      /* K */
    int32_t pages;            /* P: row length of rt */
    const int32_t* rt;        /* [batch, pages] */
    int32_t* ft;              /* [batch, ft_cols] */
    int32_t ft_cols;
    const int32_t* tail_rows; /* [batch] */
    int32_t capacity;
    int32_t fill_table;
} v1_route_args;
int v1_route(const v1_route_args* a, void* stream);

/* ------------------------------------------------------------------------
 * fused.topk: in-place sink/tail mask, exact Top-T (T <= 2048) over the
 * first fine_lens[b] candidates of each row, and the raw -> logical ->
 * physical mapping epilogue with optional x4 expansion.
 * Replaces V1QueryKernel::topk
 *   sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:181-220 (kernel :62-153).
 * Selection order: score descending, ties toward the LOWER candidate index;
 * -0.0 equals +0.0.  Each output row lists the selected candidates in
 * ascending candidate index, then -1 padding.
 * ---------------------------------------------------------------------- */
typedef struct {
    float* scores;             /* [batch, cols], row stride score_stride; masked in place */
    int64_t score_stride;
    int32_t batch;
    int32_t cols;
    const int32_t* fine_lens;  /* [batch] */
    const int32_t* members;    /* [member_pages, 64] */
    int64_t member_pages;
    const int32_t* rt;         /* [batch, pages] */
    const int32_t* nt;         /* [batch, pages] */
    int32_t pages;
    const void* selected;      /* [batch, take_stride] int32 or int64 */
    int32_t selected_bits;
    int32_t take_stride;
    const int32_t* lens;       /* [batch] */
    const int32_t* takes;      /* [batch] */
    int32_t* physical;         /* [batch, topk] (written when physical_output) */
    int32_t* logical;          /* [batch, topk] */
    int32_t* raw;              /* [batch, topk] (written when physical_output) */
    int32_t topk;
    int32_t window;
    int32_t mask;
    int32_t* expanded;         /* [batch, expansion_stride] or NULL */
    int32_t expansion_stride;  /* 0 or 4*topk+64 */
    int32_t physical_output;
    int32_t bucket_from_rank;
    const int32_t* fine_table; /* [batch, fine_table_cols] */
    int32_t fine_table_cols;
    int32_t direct_fine;
    void* workspace;           /* split rows: >= v1_topk_workspace() bytes (0 when no row is split) */
    int64_t workspace_bytes;
} v1_topk_args;
int64_t v1_topk_workspace(int32_t batch, int32_t cols, int32_t topk);
int v1_topk(const v1_topk_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Top-T with page-table transform (rows of any length, any batch):
 *   out = raw < 0 ? -1 : (page_table[b, raw >> page_bits] << page_bits) | (raw & mask)
 * Replaces TopKKernel::transform / topk_transform_512_v2
 *   sglang/kernels/jit/csrc/deepseek_v4/topk_v2.cuh:352-460,
 *   sglang/kernels/jit/include/sgl_kernel/deepseek_v4/topk_impl.cuh:156-190.
 * A work-group selects over up to 40960 columns; longer rows (and, in
 * batches of fewer than 512 rows, rows over 32768 columns) are split over
 * several work-groups, and `workspace` (device memory, >= v1_topk_workspace()
 * bytes) then holds the per-segment candidates.
 * ---------------------------------------------------------------------- */
typedef struct {
    const float* scores;        /* [batch, cols], row stride score_stride */
    int64_t score_stride;
    int32_t batch;
    int32_t cols;
    const int32_t* seq_lens;    /* [batch] */
    const int32_t* page_table;  /* [batch, page_table_cols], row stride page_table_stride */
    int64_t page_table_stride;
    int32_t page_table_cols;    /* entries past it map to -1 */
    int32_t page_bits;
    int32_t* page_indices;      /* [batch, topk] */
    int32_t* raw_indices;       /* [batch, topk] or NULL */
    int32_t topk;
    void* workspace;
    int64_t workspace_bytes;
} v1_topk_transform_args;
int v1_topk_transform(const v1_topk_transform_args* a, void* stream);

/* ------------------------------------------------------------------------
 * FP8 paged MQA index logits (the DeepGEMM fp8_paged_mqa_logits contract):
 *   logits[r, j] = sum_h w[r,h] * ReLU(sum_d q[r,h,d] * k[j,d]) * s_k[j]
 * for j < context_lens[r]; k / s_k come from native pages through
 * block_table[r, j / 64].  block_table_stride == 0 means every row shares one
 * table (a prefill chunk of one request); rows are then tiled together so that
 * each key page is staged once per row tile.  Columns in
 * [context_lens[r], max_context_len) are set to -inf when clean_logits.
 * Formula: sglang/srt/layers/attention/v1_deepseek/kernels.py:248-320,
 * experiments/fine_pool_shared_20261021/test_and_bench.py:37; call sites
 * sglang/srt/layers/attention/v1_deepseek/runtime.py:434-444, 538-548.
 * ---------------------------------------------------------------------- */
typedef struct {
    const uint8_t* q;            /* [rows, heads, 128] e4m3fn */
    const uint8_t* kv_pages;     /* [blocks, 8448] */
    int64_t kv_blocks;
    const float* weights;        /* [rows, heads] */
    const int32_t* context_lens; /* [rows] */
    const int32_t* block_table;  /* [rows, max_blocks], row stride block_table_stride */
    int64_t block_table_stride;
    int32_t max_blocks;
    float* logits;               /* [rows, logits_stride] */
    int64_t logits_stride;
    int32_t max_context_len;
    int32_t rows;
    int32_t heads;               /* 1..64 */
    int32_t relu;                /* 1: DSA ReLU rule; 0: signed scores */
    int32_t clean_logits;
    void* workspace;             /* shared tables: >= v1_score_workspace(rows, max_context_len) bytes;
                                    per-row tables: optional, see v1_score_tables_workspace */
    int64_t workspace_bytes;
} v1_score_args;
/* Workspace of the shared-table path: per-query records, a work counter and,
 * for the ReLU rule, per-row bitmaps of pages rescored exactly (keys whose
 * fast value is within rounding of zero get the direct ReLU sum, so keys with
 * no positive head dot score exactly 0, as kernels.py:310-313 gives). */
int64_t v1_score_workspace(int32_t rows, int32_t max_context_len);
/* Per-row block tables (block_table_stride != 0) of more than 512 rows and
 * more than 16 heads with max_context_len <= 65536: given a 256-byte aligned
 * workspace of at least
 * this many bytes (0 when the shape does not qualify), v1_score plans each
 * group of 8 rows over the union of their table pages and stages every page
 * once for the group (the rows of one prefill chunk share most pages, as the
 * fine tables of runtime.py:538-548 do); groups sharing less than two rows
 * per page, and calls without the workspace, score each row on its own. */
int64_t v1_score_tables_workspace(int32_t rows, int32_t max_context_len);
/* Workspace bytes for per-row tables scored page-major (0: not taken).  For
 * more than 512 rows over a pool of at most 32768 pages whose dense pair
 * table (rows x kv_blocks x 4 bytes) fits 64 MiB, e.g. a prefill chunk's fine
 * tables over one request's pages: each work-group stages 8 listed pool pages
 * in LDS once and scores every row of a 64-row block that lists them.  v1_score takes
 * this form for more than 16 heads when its workspace holds this many bytes (checked before the
 * page-union plan of v1_score_tables_workspace); the values are those of the
 * row-by-row kernel, bit for bit.  No counterpart in the reference, which
 * scores each row's table on its own (runtime.py:538-548). */
int64_t v1_score_pages_workspace(int32_t rows, int32_t max_context_len, int64_t kv_blocks);
/* 0 keeps v1_score off the page-major form (then the page-union plan takes
 * per-row tables of large batches), 1 (the default) allows it; process-wide,
 * the previous setting goes to *previous (if not NULL).  No counterpart in the
 * reference: a switch for tests and measurements. */
int v1_score_page_major(int32_t enable, int32_t* previous);
int v1_score(const v1_score_args* a, void* stream);
/* v1_score without a caller workspace and without any allocation: the
 * shared-table path's scratch is a static 16 MiB device array per GPU
 * (v1_score_noalloc_capacity() bytes), so rows * max_context_len must fit
 * v1_score_workspace(rows, max_context_len) <= that, else V1_ERR_INVALID.
 * a->workspace is ignored.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops).  Every call on a GPU shares that GPU's array, so calls that overlap
 * on one GPU race; per-row tables need no scratch and do not touch it. */
int64_t v1_score_noalloc_capacity(void);
int v1_score_noalloc(const v1_score_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Scoring without DeepGEMM: the reference's Triton fallbacks, used when
 * DeepGEMM is absent or the query optimisations are off
 * (sglang/srt/layers/attention/v1_deepseek/runtime.py:450-466, 565-590).
 *
 * reduce_centers (kernels.py:475-486): scores[r, p] = max of
 * logits[r, 8p .. 8p+7] for p < max(lens[r]-1, 0) / 1024 * 16, else -inf;
 * scores is [rows, maxp].
 * ---------------------------------------------------------------------- */
int v1_reduce_centers(const float* logits, int64_t logits_stride, const int32_t* lens, float* scores,
                      int32_t rows, int32_t maxp, void* stream);

/* coarse (kernels.py:182-221): center page table[r, b] holds the 64 centers
 * of pages 8b..8b+7; a page scores the max of its 8 centers'
 * sum_h w relu(q . c) s_c for pages below max(lens[r]-1, 0) / 1024 * 16 (at
 * most maxp), else -inf.  Runs as center logits (v1_score over the row's
 * centers) reduced by v1_reduce_centers, in the caller's workspace. */
typedef struct {
    const uint8_t* q;             /* [rows, heads, 128] e4m3fn */
    const float* weights;         /* [rows, heads] */
    const uint8_t* centers;       /* center pages [center_blocks, 8448] */
    int64_t center_blocks;
    const int32_t* table;         /* [rows, maxp / 8] center pages, row stride table_stride (0: shared) */
    int64_t table_stride;
    const int32_t* lens;          /* [rows] tokens */
    float* scores;                /* [rows, maxp] */
    int32_t rows;
    int32_t heads;
    int32_t maxp;                 /* multiple of 8 */
    int32_t relu;
    void* workspace;              /* >= v1_coarse_workspace(rows, maxp, table_stride) bytes, 256-byte aligned */
    int64_t workspace_bytes;
} v1_coarse_args;
int64_t v1_coarse_workspace(int32_t rows, int32_t maxp, int64_t table_stride);
int v1_coarse(const v1_coarse_args* a, void* stream);

/* fine (kernels.py:248-320): scores[r, i] for i < width.  i < take * 64 is
 * slot i % 64 of fine page rt[r, selected[r, i / 64]], kept when its logical
 * position members[page][slot] lies in [sink, tail) and below lens[r]; the
 * next sink + n - tail candidates are the sink and tail tokens read from
 * native pages nt[r, logical / 64]; -inf elsewhere (also for ranks, pages or
 * logical pages outside their tables).  sink = min(n, sink_cap), tail as the
 * reference's query_lengths. */
typedef struct {
    const uint8_t* q;             /* [rows, heads, 128] e4m3fn */
    const float* weights;         /* [rows, heads] */
    const uint8_t* fine_pages;    /* fine pool [fine_blocks, 8448] */
    int64_t fine_blocks;
    const uint8_t* native_pages;  /* native pool [native_blocks, 8448] */
    int64_t native_blocks;
    const int32_t* members;       /* [fine_blocks, 64] logical positions */
    const int32_t* rt;            /* [rows, maxp] reordered table */
    const int32_t* nt;            /* [rows, np] native table */
    const void* selected;         /* [rows, take_stride] ranks, int32 or int64 */
    int32_t selected_bits;
    const int32_t* lens;          /* [rows] tokens */
    const int32_t* takes;         /* [rows] */
    float* scores;                /* [rows, width] */
    int32_t rows;
    int32_t heads;
    int32_t maxp;
    int32_t np;
    int32_t take_stride;
    int32_t width;
    int32_t sink;
    int32_t window;
    int32_t relu;
} v1_fine_args;
int v1_fine(const v1_fine_args* a, void* stream);

/* ------------------------------------------------------------------------
 * _gather_slots: logical -> req[logical] -> K and V rows of one head into
 * contiguous [rows, top, 128] outputs; ids < 0 give zero rows.
 * Replaces sglang/srt/layers/attention/v1_native/kernels.py:62-77 (_gather_slots)
 * as launched by GatherWorkspace.gather (:102-111).  Strides in elements.
 * ids >= req_len or req entries outside [0, pool_slots) give zero rows.
 * ---------------------------------------------------------------------- */
int v1_gather_slots(const void* k_pool, const void* v_pool, int64_t pool_slots, int32_t elem_bytes,
                    int64_t ks0, int64_t ks1, int64_t ks2,
                    int64_t vs0, int64_t vs1, int64_t vs2, int32_t head,
                    const int32_t* req, int64_t req_len, const int32_t* ids, int64_t ids_stride,
                    int32_t rows, int32_t top, void* k_out, void* v_out, void* stream);

/* ------------------------------------------------------------------------
 * Byte-row gather (the _gather_slots contract generalised to opaque rows,
 * e.g. 656-byte MLA latent rows): for t = r*top + i, id = ids[r*ids_stride+i];
 *   id < 0            -> out row t = zeros
 *   map == NULL       -> physical = id
 *   otherwise         -> physical = (map[r*map_stride + (id >> map_shift)] << map_shift)
 *                                   | (id & ((1 << map_shift) - 1))
 * and out[t*row_bytes ...] = pool[physical*pool_stride_bytes ...].
 * map_stride == 0 shares one map (the reference REQ vector) across rows;
 * map_len is the number of entries of one map row.  An id whose map entry or
 * physical row falls outside [0, map_len) / [0, pool_rows) yields a zero row
 * (the reference leaves such ids undefined).
 * ---------------------------------------------------------------------- */
int v1_gather_rows(const void* pool, int64_t pool_rows, int64_t row_bytes, int64_t pool_stride_bytes,
                   const int32_t* map, int64_t map_len, int64_t map_stride, int32_t map_shift,
                   const int32_t* ids, int64_t ids_stride, int32_t rows, int32_t top,
                   void* out, void* stream);

/* ------------------------------------------------------------------------
 * _sort: per group g of n keys, out[g*n + i] = perm[g*n + pos_i] where pos
 * orders the group's keys descending, ties by ascending position.
 * fp32 keys (-0.0 == +0.0):  sglang/srt/layers/attention/v1_native/fused_grouping.py:64-76
 * (only when *flag < 0; head h uses offset h*head_stride).  int64 keys are the
 * same rule over signed 64-bit keys.  perm and out must not overlap.
 * n is a power of two in [2, 4096].
 * ---------------------------------------------------------------------- */
int v1_sort_f32(const int32_t* perm, int32_t* out, const float* keys, const int32_t* flag,
                int32_t n, int32_t groups, int32_t heads, int64_t head_stride, void* stream);
int v1_sort_i64(const int32_t* perm, int32_t* out, const int64_t* keys, const int32_t* flag,
                int32_t n, int32_t groups, void* stream);

/* ------------------------------------------------------------------------
 * Index-build producer (the pages the query path reads): per 1024-token
 * bucket of 16 native pages, unit vectors, a balanced cosine bisection into
 * groups of 8, then the permuted pages, member map and FP8 centers.
 * Arithmetic: every 128-wide fp32 sum keeps four partial sums (dims d = r
 * mod 4, ascending d, no fused multiply-add) then (p0 + p1) + (p2 + p3);
 * unit_d = c_d * (s / max(||x||, 1e-12)); center means add the 8 members in
 * order, times 1/8.  K / KS and TMP / TMPS and CENTERS / CS are byte / fp32
 * views of the same pages, indexed as in the reference.
 * ---------------------------------------------------------------------- */
/* initialize: sglang/srt/layers/attention/v1_deepseek/kernels.py:9-30 (grid
 * (programs,), 16 tokens each; FLAG = meta[2] ? -1 : 0). */
int v1_build_initialize(const void* K, const float* KS, const int32_t* table, const int32_t* meta, float* unit,
                        int32_t* perm, int32_t* flag, int32_t programs, void* stream);
/* _dots: sglang/srt/layers/attention/v1_native/fused_grouping.py:38-52 (grid
 * (programs, heads), 16 positions each; runs when *flag < 0). */
int v1_group_dots(const float* U, const int32_t* P, const int32_t* A, float* S, const int32_t* flag, int32_t N,
                  int32_t start, int32_t mode, int32_t programs, int32_t heads, void* stream);
/* _anchor: fused_grouping.py:54-61 (grid (groups, heads); leftmost minimum). */
int v1_group_anchor(const int32_t* P, int32_t* A, const float* S, const int32_t* flag, int32_t N, int32_t slot,
                    int32_t groups, int32_t heads, void* stream);
/* assemble: sglang/srt/layers/attention/v1_deepseek/kernels.py:33-54 (grid
 * (pages, groups) = (16, 8); runs when meta[2] != 0). */
int v1_build_assemble(const void* K, const float* KS, const int32_t* table, const int32_t* meta,
                      const int32_t* ids, void* tmp, float* tmps, void* centers, float* cs, int32_t* map,
                      int32_t pages, int32_t groups, void* stream);
/* The chain initialize -> 7 x (3 _dots, 2 _anchor, _sort) -> assemble of
 * sglang/srt/layers/attention/v1_deepseek/runtime.py:171-216 for a batch of
 * buckets in one launch: bucket b reads pages tables[b*16 .. b*16+15] of the
 * pool and writes perm [b, 1024] (token order, 0..1023), tmp [b, 16 pages],
 * mapping [b, 1024] = starts[b] + perm and centers [b, 2 pages].  Identical
 * results to the chain of the entry points above.  Table entries outside
 * [0, pool_pages) read page 0. */
int v1_build_buckets(const void* pool, int64_t pool_pages, const int32_t* tables, const int32_t* starts,
                     int32_t buckets, int32_t* perm, void* tmp, int32_t* mapping, void* centers, void* stream);

/* ------------------------------------------------------------------------
 * Page manager: sglang/srt/layers/attention/v1_deepseek/kernels.py:57-179
 * (fingerprint 57-69, match_pages 72-113, allocate 116-131, publish 134-167,
 * release 170-179).  Each call handles one 16-page bucket record gated by
 * meta[2] (active); meta[1] is the lease.  page_bytes is 8448 for the
 * reference pages.  status (int32, may be NULL) receives bit 0 when
 * allocate finds the free stack exhausted (the reference device_assert).
 * ---------------------------------------------------------------------- */
int v1_fingerprint(const uint8_t* tmp, const int32_t* map, const int32_t* meta, int64_t* hash,
                   int32_t pages, int64_t page_bytes, void* stream);
int v1_match_pages(const uint8_t* tmp, const int32_t* map, const int64_t* hash, const int32_t* meta,
                   const uint8_t* fine, const int32_t* members, const int64_t* hashes,
                   const int32_t* refs, int32_t* match, int32_t pages, int32_t capacity,
                   int64_t page_bytes, void* stream);
int v1_allocate(const int32_t* meta, const int32_t* match, int32_t* free_stack, int32_t* count,
                int32_t* refs, int32_t* tables, uint8_t* fresh, int32_t pages, int32_t* status,
                void* stream);
int v1_publish(const uint8_t* tmp, const uint8_t* centers_src, const int32_t* map, const int64_t* hash,
               const int32_t* meta, const int32_t* tables, const uint8_t* fresh, uint8_t* fine,
               uint8_t* centers, int32_t* members, int64_t* hashes, int32_t pages,
               int64_t page_bytes, void* stream);
int v1_release(const int32_t* table, int32_t* refs, int32_t* free_stack, int32_t* count,
               int32_t pages, void* stream);

/* ------------------------------------------------------------------------
 * Device-wide stable sort of (uint64 key, uint32 value) pairs, ascending by
 * key, equal keys in input order: the int64-key grouping of _sort
 * (sglang/srt/layers/attention/v1_native/fused_grouping.py:64-76) over a whole
 * batch of page keys rather than one 4096-key group.  key_bits: the low bits
 * that may differ (64 for arbitrary keys).  Outputs must not alias inputs.
 * ---------------------------------------------------------------------- */
int64_t v1_sort_pairs_u64_workspace(int64_t n);
int v1_sort_pairs_u64(const uint64_t* keys, const uint32_t* vals, uint64_t* keys_out,
                      uint32_t* vals_out, int64_t n, int32_t key_bits, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Batched page manager: match_pages -> allocate -> publish for a batch of
 * requests (kernels.py:72-167, host order runtime.py:230-270), and release
 * (kernels.py:170-179) of a list of pages.  The results equal running the
 * per-lease kernels request after request:
 *   - entry e (page bytes tmp[e], int64 key keys[e], request req[e], req
 *     non-decreasing) takes the lowest live page with equal key and equal
 *     bytes; live = refs > 0 before the batch or published by an earlier
 *     request of the batch; entries of one request never match each other;
 *   - unmatched entries take free_stack[count - 1 - rank] in entry order;
 *   - table[e] = page, refs[page] += 1, fresh pages get the bytes and key.
 * The key stands in for the reference's (h0, h1) fingerprint.  Release
 * decrements in list order; a page that reaches 0 is pushed on the free stack
 * in list order.  A batch that fails (status bits below, OR-ed into *status)
 * leaves pool, keys, refs, free stack and count unchanged.  page_bytes is a
 * multiple of 16 (41984 for 64 MLA rows of 656 bytes, 8448 for native pages).
 * ---------------------------------------------------------------------- */
#define V1_STATUS_EXHAUSTED 1   /* free stack smaller than the fresh pages needed */
#define V1_STATUS_COLLISIONS 2  /* more than 4096 entries whose key collides with other bytes */
#define V1_STATUS_BAD_ORDER 4   /* req decreases */
#define V1_STATUS_UNDERFLOW 8   /* release of a page whose count is 0, or a page id out of range */
#define V1_STATUS_BAD_STATE 16  /* count outside [0, capacity] or a free-stack page id out of range */
int64_t v1_page_insert_workspace(int32_t capacity, int32_t n);
int v1_page_insert(uint8_t* pool, int64_t* pool_keys, int32_t* refs, int32_t* free_stack,
                   int32_t* count, int32_t capacity, int64_t page_bytes, const int64_t* keys,
                   const uint8_t* tmp, const int32_t* req, int32_t n, int32_t* table,
                   int32_t* status, void* workspace, int64_t workspace_bytes, void* stream);
int64_t v1_page_release_workspace(int32_t capacity, int32_t n);
int v1_page_release(const int32_t* pages, int32_t n, int32_t* refs, int32_t* free_stack,
                    int32_t* count, int32_t capacity, int32_t* status, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Query metadata, fine page tables and shared tail staging:
 * query_metadata    sglang/srt/layers/attention/v1_deepseek/kernels.py:568-591
 * query_lengths     kernels.py:224-245
 * fine_table_shared kernels.py:488-514   (tail_rows == NULL: fine_table :379-404)
 * stage_tail_shared kernels.py:518-564   (tail_rows == NULL: stage_tail :407-441)
 * mask_fine         kernels.py:444-472
 * output_ids        kernels.py:323-376
 * ---------------------------------------------------------------------- */
int v1_query_metadata(const int32_t* lens, const int32_t* nt, int32_t* fine_lens, int32_t* takes,
                      int32_t* dg_lens, int32_t* center_lens, int32_t* tail_rows, int32_t rows,
                      int32_t np, int32_t topk, int32_t num, int32_t den, int32_t sink,
                      int32_t window, void* stream);
int v1_query_lengths(const int32_t* lens, int32_t* fine_lens, int32_t* takes, int32_t rows,
                     int32_t topk, int32_t num, int32_t den, int32_t sink, int32_t window,
                     void* stream);
int v1_fine_table(const int32_t* rt, const void* selected, int32_t selected_bits,
                  const int32_t* takes, int32_t* ft, const int32_t* tail_rows, int32_t rows,
                  int32_t capacity, int32_t maxp, int32_t take_stride, int32_t fp,
                  int32_t scratch, void* stream);
int v1_stage_tail(const uint8_t* native, const int32_t* nt, const int32_t* lens, uint8_t* fine,
                  const int32_t* tail_rows, int32_t rows, int32_t capacity, int32_t np,
                  int32_t scratch, int32_t sink, int32_t window, int64_t native_pages,
                  int64_t fine_pages, void* stream);
/* stage_tail / stage_tail_shared (kernels.py:518-564, :407-441) over pages of
 * 64 rows of row_bytes each (656 for MLA latent rows): the same owner, slot and
 * zero-fill rule, one contiguous row per token. */
int v1_stage_tail_rows(const uint8_t* native, const int32_t* nt, const int32_t* lens, uint8_t* fine,
                       const int32_t* tail_rows, int32_t rows, int32_t capacity, int32_t np,
                       int32_t scratch, int32_t sink, int32_t window, int64_t native_pages,
                       int64_t fine_pages, int32_t row_bytes, void* stream);
int v1_mask_fine(float* scores, int64_t score_stride, const void* selected, int32_t selected_bits,
                 const int32_t* rt, const int32_t* members, const int32_t* lens,
                 const int32_t* takes, int32_t rows, int32_t maxp, int32_t take_stride,
                 int32_t width, int32_t sink, int32_t window, void* stream);
int v1_output_ids(const int32_t* raw, const float* scores, int64_t score_stride,
                  const int32_t* members, const int32_t* rt, const int32_t* nt,
                  const void* selected, int32_t selected_bits, const int32_t* lens,
                  const int32_t* takes, int32_t* out, int32_t* logical, const int32_t* ft,
                  int32_t rows, int32_t maxp, int32_t np, int32_t take_stride, int32_t width,
                  int32_t topk, int32_t sink, int32_t window, int32_t map_physical,
                  int32_t direct_fine, int32_t fp, void* stream);

/* expand_logical, sglang/srt/layers/attention/v1_deepseek/kernels.py:594-600
 * (the unfused C4 x4 expansion, runtime.py:638-641): out[r, j] = 4*logical[r, j/4]
 * + j%4 for j < 4*topk and logical >= 0, else -1, for columns j < cols (the
 * reference's min(STRIDE, BLOCK)); logical is [rows, topk] contiguous, out rows
 * are `stride` ints apart (stride >= cols). */
int v1_expand_logical(const int32_t* logical, int32_t* out, int32_t rows, int32_t topk, int64_t stride,
                      int32_t cols, void* stream);
/* ------------------------------------------------------------------------
 * Shared sink + tail staging with a published index end (one request's causal
 * chunk, rows with non-decreasing lengths; no host reads, graph-capturable):
 * stage_tail_published  experiments/tail_union_lab_20261021/baseline_published.py:4-61
 *                       (stage_tail_shared with the tail starting at indexed_end)
 * stage_union           experiments/tail_union_lab_20261021/union.py:10-42
 * union_tables          experiments/fine_pool_shared_20261021/kernels.py:13-35 (tables)
 * union_normalize       kernels.py:38-59 (normalize)
 * union_map_topk        kernels.py:62-76 (map_topk)
 * Row bounds: s = min(n, sink), t = max(s, min(min(max(end, 0), n),
 * max(s, n - window))), count = s + n - t.  stage_union copies the union of all
 * rows' sink and tail pages once into dst (pages past its capacity are not
 * copied), writes meta [rows, 3] = (s, t, count) and desc = (sp, tp, ep, total).
 * ---------------------------------------------------------------------- */
/* Split scoring of the shared chunk (no counterpart call in the reference: its
 * scores come from per-row tables, kernels.py:13-59; these give the same
 * canonical candidate vector from two shared-table scorings): union_spans
 * writes each row's span in union coordinates (positions up * 64 + slot,
 * up = lp for sink pages and sp + lp - tp for tail pages); normalize_split
 * builds the canonical scores from hist [rows, >= 64 * history pages]
 * (position page * 64 + slot) and uni [rows, >= span], with normalize's masks. */
int v1_union_spans(const int32_t* lens, const int32_t* indexed_end, const int32_t* desc, int32_t* spans,
                   int32_t rows, int32_t sink, int32_t window, void* stream);
int v1_union_normalize_split(const float* hist, int64_t hist_stride, int32_t hist_cols, const float* uni,
                             int64_t uni_stride, int32_t uni_cols, const int32_t* lens,
                             const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                             const int32_t* members, int64_t members_pages, const int32_t* desc, float* out,
                             int32_t rows, int32_t max_take, int32_t width, int32_t sink, int32_t window,
                             void* stream);
int v1_stage_tail_published(const uint8_t* native, const int32_t* nt, const int32_t* lens,
                            const int32_t* indexed_end, uint8_t* fine, const int32_t* tail_rows,
                            int32_t rows, int32_t capacity, int32_t np, int32_t scratch, int32_t sink,
                            int32_t window, int64_t native_pages, int64_t fine_pages, void* stream);
int v1_stage_union(const void* src, int64_t src_pages, const int32_t* nt, int32_t nt_len,
                   const int32_t* lens, int32_t rows, const int32_t* indexed_end, void* dst,
                   int32_t dst_pages, int32_t* meta, int32_t* desc, int32_t sink, int32_t window,
                   void* stream);
int v1_union_tables(const int32_t* lens, const int32_t* indexed_end, const int32_t* takes,
                    const int32_t* selected, const int32_t* desc, int32_t* ft, int32_t* dg_lens,
                    int32_t* clens, int32_t rows, int32_t cap, int32_t max_take, int32_t scratch,
                    int32_t fp, int32_t sink, int32_t window, int32_t shared, void* stream);
int v1_union_normalize(const float* raw, int64_t raw_stride, int32_t raw_cols, const int32_t* lens,
                       const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                       const int32_t* members, int64_t members_pages, float* out, int32_t rows,
                       int32_t max_take, int32_t width, int32_t sink, int32_t window, int32_t shared,
                       void* stream);
/* values == NULL: the value of id i is scores[r * score_stride + i] (the
 * canonical scores the Top-K selected from; -inf past score_cols). */
int v1_union_map_topk(const void* ids, int32_t ids_bits, const float* values, const float* scores,
                      int64_t score_stride, int32_t score_cols, const int32_t* lens,
                      const int32_t* indexed_end, const int32_t* takes, const int32_t* selected,
                      const int32_t* members, int64_t members_pages, const int32_t* nt, int32_t nt_len,
                      int32_t* logical, int32_t* slots, int32_t rows, int32_t max_take, int32_t top,
                      int32_t sink, int32_t window, void* stream);
/* ------------------------------------------------------------------------
 * Decode attention over the gathered workspace (the consumer after the slot
 * gather): sglang/srt/layers/attention/v1_native/backend.py:306-315 calls
 * flash_attn_with_kvcache(q[:, None], kg, vg, causal=False, softmax_scale)
 * on GatherWorkspace rows.  bf16 q [batch, heads_q, 128], k / v [batch, keys,
 * heads_kv, 128] (element strides, inner dim contiguous, 16-byte aligned),
 * heads_q / heads_kv <= 4 query heads per KV head, keys * group <= 12288;
 * out[b, h] (bf16) = softmax over the first seqlens[b] keys (all keys when
 * seqlens is NULL; zeros for a row without keys) of scale * q . k, times v.
 * ---------------------------------------------------------------------- */
int v1_decode_attention(const void* q, int64_t q_batch, int64_t q_head, const void* k, int64_t k_batch,
                        int64_t k_token, int64_t k_head, const void* v, int64_t v_batch, int64_t v_token,
                        int64_t v_head, const int32_t* seqlens, void* out, int64_t o_batch, int64_t o_head,
                        int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t keys, float scale,
                        void* stream);
/* The same attention with the gather folded in: key j of row b is slot
 * req[ids[b * ids_stride + j]] of KV head `head` of the pools (k_pool[slot *
 * k_slot + head * k_head + d]), an id < 0 or >= req_len or a slot outside
 * [0, pool_slots) being a zero key and value (GatherWorkspace's rule,
 * sglang/srt/layers/attention/v1_native/kernels.py:62-77): equal, bit for
 * bit, to v1_gather_slots followed by v1_decode_attention, without the
 * workspace.  heads_q <= 4 query heads, keys * (heads_q + 1) <= 12288. */
int v1_decode_attention_slots(const void* q, int64_t q_batch, int64_t q_head, const void* k_pool,
                              int64_t k_slot, int64_t k_head, const void* v_pool, int64_t v_slot,
                              int64_t v_head, int64_t pool_slots, int32_t head, const int32_t* req,
                              int64_t req_len, const int32_t* ids, int64_t ids_stride, void* out,
                              int64_t o_batch, int64_t o_head, int32_t rows, int32_t heads_q, int32_t keys,
                              float scale, void* stream);
#ifdef __cplusplus
}
#endif
#endif /* V1IDX_H */
