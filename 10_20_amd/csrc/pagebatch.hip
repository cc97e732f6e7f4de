// Batched page manager: match -> allocate -> publish for a whole batch of
// requests, and the matching release, with the result of running the
// reference's per-lease kernels request after request
// (sglang/srt/layers/attention/v1_deepseek/kernels.py:72-179, host order
// sglang/srt/layers/attention/v1_deepseek/runtime.py:230-270):
//
//  * an entry (one page of request r) takes the lowest-numbered live page with
//    its key and equal bytes (match_pages :72-113); live means refs > 0, either
//    before the batch or published by a request before r;
//  * the entries of one request are not matched against each other: each
//    unmatched one takes a fresh page (allocate :116-131), popped from the free
//    stack in request order, free[count - 1 - rank];
//  * every entry adds one reference to its page; fresh pages receive the
//    entry's bytes and key (publish :134-167);
//  * release (:170-179) of a list of pages: decrements in list order, a page
//    dies at the decrement that takes its count from 1 to 0, dead pages are
//    pushed on the free stack in that order.
//
// The int64 key plays the part of the reference's (h0, h1) fingerprint
// (:57-69); the byte comparison guards key collisions.
//
// Parallel form.  Live pages (in page order) and entries (in request order)
// are sorted together by key with a stable radix sort, so every key group
// starts with its lowest live page, else with its first entry: the group's
// representative.  An entry whose bytes equal the representative's resolves
// at once: a live representative is its page; otherwise the entries of the
// representative's request are fresh and later entries take the lowest of
// those fresh pages.  Entries whose bytes differ from their representative
// (key collisions) are resolved by one wave, in request order, against the
// group's live pages and the earlier colliding entries.  Fresh ranks are one
// prefix sum.  A batch that would exhaust the free stack, holds more than
// kSlowMax colliding entries or has decreasing request ids changes nothing
// and reports it in the status word.
#include "common.h"

namespace v1 {
namespace {

constexpr uint32_t kPageTag = 0x80000000u;  // sort value of a live page: page | kPageTag
constexpr uint32_t kPad = 0x7fffffffu;      // sort value of padding (sorts after every real pair)
constexpr int32_t kClassLive = 0x40000000;  // class of an entry: live page | kClassLive, else its first entry
constexpr int32_t kSlowMax = 4096;          // colliding entries resolved per batch
constexpr int kThreads = 256;

struct InsertState {
    uint8_t* pool;        // [cap, page_bytes]
    int64_t* pool_keys;   // [cap]
    int32_t* refs;        // [cap]
    int32_t* free_stack;  // [cap]
    int32_t* count;       // scalar
    int32_t cap;
    int64_t page_bytes;
    const int64_t* keys;  // [n]
    const uint8_t* tmp;   // [n, page_bytes]
    const int32_t* req;   // [n], non-decreasing
    int32_t n;
    int32_t* table;       // [n] out
    int32_t* status;      // scalar, bits OR-ed in
    // workspace
    uint32_t* live_flag;  // [cap]
    uint32_t* live_off;   // [cap]
    uint32_t* nlive;
    uint64_t* skeys;      // [m]  m = cap + n
    uint32_t* svals;      // [m]
    uint64_t* okeys;      // [m]
    uint32_t* ovals;      // [m]
    uint32_t* head;       // [m]
    uint32_t* gid;        // [m]
    uint32_t* start;      // [m] group id -> first position
    uint32_t* ngroups;
    int32_t* pos_of;      // [n] entry -> sorted position
    int32_t* cls;         // [n]
    uint32_t* fresh;      // [n]
    uint32_t* rank;       // [n]
    uint32_t* nfresh;
    int32_t* fresh_list;  // [n] rank -> entry
    int32_t* page_of;     // [n] fresh page of a fresh entry
    int32_t* class_min;   // [n] lowest fresh page of a batch class
    int32_t* slow;        // [kSlowMax]
    uint32_t* nslow;
    uint32_t* abort;      // nonzero: leave the pool unchanged
};

__device__ __forceinline__ const uint8_t* bytes_of(const InsertState& s, uint32_t val) {
    return (val & kPageTag) ? s.pool + (int64_t)(val & ~kPageTag) * s.page_bytes
                            : s.tmp + (int64_t)val * s.page_bytes;
}

// One wave: are the two pages equal?  page_bytes is a multiple of 16 and both
// pages are 16-byte aligned; eight 16-byte loads per lane are in flight.
__device__ bool wave_equal(const uint8_t* a, const uint8_t* b, int64_t bytes) {
    const int l = __lane_id();
    const uint4* x = reinterpret_cast<const uint4*>(a);
    const uint4* y = reinterpret_cast<const uint4*>(b);
    const int64_t chunks = bytes >> 4;
    uint32_t diff = 0;
    int64_t c = l;
    for (; c + 3 * kWave < chunks; c += 4 * kWave) {
        uint4 xa[4], ya[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            xa[u] = x[c + u * kWave];
            ya[u] = y[c + u * kWave];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            diff |= (xa[u].x ^ ya[u].x) | (xa[u].y ^ ya[u].y) | (xa[u].z ^ ya[u].z) | (xa[u].w ^ ya[u].w);
    }
    for (; c < chunks; c += kWave) {
        const uint4 p = x[c], q = y[c];
        diff |= (p.x ^ q.x) | (p.y ^ q.y) | (p.z ^ q.z) | (p.w ^ q.w);
    }
    return __ballot(diff != 0) == 0;
}

// gid is the exclusive scan of head: a head's own group, else the last head's
__device__ __forceinline__ uint32_t group_of(const uint32_t* gid, const uint32_t* head, int64_t i) {
    return gid[i] + head[i] - 1u;
}

__global__ __launch_bounds__(kThreads) void pb_live_flags(InsertState s) {
    const int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (p < s.cap) s.live_flag[p] = s.refs[p] > 0 ? 1u : 0u;
    if (p == 0) {
        *s.nslow = 0;
        *s.abort = 0;
    }
}

// sort input: [live pages in page order | entries in request order | padding]
__global__ __launch_bounds__(kThreads) void pb_sort_input(InsertState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const uint32_t nlive = *s.nlive;
    if (i < s.cap && s.live_flag[i]) {
        const uint32_t at = s.live_off[i];
        s.skeys[at] = (uint64_t)s.pool_keys[i];
        s.svals[at] = (uint32_t)i | kPageTag;
    }
    if (i < s.n) {
        const int64_t at = (int64_t)nlive + i;
        s.skeys[at] = (uint64_t)s.keys[i];
        s.svals[at] = (uint32_t)i;
        s.class_min[i] = 0x7fffffff;
        if (i + 1 < s.n && s.req[i] > s.req[i + 1]) {
            atomicOr(s.status, V1_STATUS_BAD_ORDER);
            atomicOr(s.abort, 1u);
        }
    }
    if (i < (int64_t)s.cap - nlive) {
        const int64_t at = (int64_t)nlive + s.n + i;
        s.skeys[at] = ~0ull;
        s.svals[at] = kPad;
    }
}

__global__ __launch_bounds__(kThreads) void pb_heads(const uint64_t* okeys, uint32_t* head, int64_t m) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < m) head[i] = (i == 0 || okeys[i] != okeys[i - 1]) ? 1u : 0u;
}

__global__ __launch_bounds__(kThreads) void pb_groups(InsertState s, int64_t m) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= m) return;
    if (s.head[i]) s.start[s.gid[i]] = (uint32_t)i;
    const uint32_t v = s.ovals[i];
    if (!(v & kPageTag) && v != kPad) s.pos_of[v] = (int32_t)i;
}

// One wave per entry: its class from the group's representative.
__global__ __launch_bounds__(kThreads) void pb_classify(InsertState s) {
    const int64_t e = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (e >= s.n) return;
    const int64_t i = s.pos_of[e];
    const uint32_t rep = s.ovals[s.start[group_of(s.gid, s.head, i)]];
    const bool same = rep == (uint32_t)e || wave_equal(bytes_of(s, (uint32_t)e), bytes_of(s, rep), s.page_bytes);
    if (__lane_id() != 0) return;
    if (!same) {
        s.cls[e] = -1;
        s.fresh[e] = 0;
        const uint32_t k = atomicAdd(s.nslow, 1u);
        if (k < (uint32_t)kSlowMax) s.slow[k] = (int32_t)e;
    } else if (rep & kPageTag) {
        s.cls[e] = (int32_t)(rep & ~kPageTag) | kClassLive;
        s.fresh[e] = 0;
    } else {
        s.cls[e] = (int32_t)rep;
        s.fresh[e] = s.req[e] == s.req[rep] ? 1u : 0u;
    }
}

// Colliding entries, one wave, in entry order: the lowest live page of the
// group with equal bytes, else the class of the earliest colliding entry with
// equal key and bytes, else a class of its own.
__global__ __launch_bounds__(kWave) void pb_slow(InsertState s, int64_t m) {
    __shared__ int32_t list[kSlowMax];
    __shared__ int32_t list_cls[kSlowMax];
    const uint32_t ns = *s.nslow;
    if (ns == 0) return;
    const int l = __lane_id();
    if (ns > (uint32_t)kSlowMax) {
        if (l == 0) {
            atomicOr(s.status, V1_STATUS_COLLISIONS);
            atomicOr(s.abort, 1u);
        }
        return;
    }
    for (uint32_t k = l; k < ns; k += kWave) list[k] = s.slow[k];
    __syncthreads();
    if (l == 0) {  // insertion order is arbitrary: sort the short list by entry
        for (uint32_t a = 1; a < ns; ++a) {
            const int32_t v = list[a];
            int32_t b = (int32_t)a - 1;
            while (b >= 0 && list[b] > v) {
                list[b + 1] = list[b];
                --b;
            }
            list[b + 1] = v;
        }
    }
    __syncthreads();
    for (uint32_t k = 0; k < ns; ++k) {
        const int32_t e = list[k];
        const int64_t i = s.pos_of[e];
        const uint64_t key = s.okeys[i];
        int32_t c = -1;
        for (int64_t j = s.start[group_of(s.gid, s.head, i)]; c < 0 && j < m && s.okeys[j] == key; ++j) {
            const uint32_t v = s.ovals[j];
            if (!(v & kPageTag)) break;  // live pages lead the group
            if (wave_equal(bytes_of(s, (uint32_t)e), bytes_of(s, v), s.page_bytes))
                c = (int32_t)(v & ~kPageTag) | kClassLive;
        }
        for (uint32_t k2 = 0; c < 0 && k2 < k; ++k2) {
            const int32_t y = list[k2];
            if (s.keys[y] != s.keys[e]) continue;
            if (wave_equal(bytes_of(s, (uint32_t)e), bytes_of(s, (uint32_t)y), s.page_bytes)) c = list_cls[k2];
        }
        if (c < 0) c = e;
        const uint32_t fr = (c & kClassLive) ? 0u : (s.req[e] == s.req[c] ? 1u : 0u);
        if (l == 0) {
            list_cls[k] = c;
            s.cls[e] = c;
            s.fresh[e] = fr;
        }
        __syncthreads();
    }
}

// fresh pages from the free stack; the lowest fresh page of every batch class
__global__ __launch_bounds__(kThreads) void pb_allocate(InsertState s) {
    const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const uint32_t need = *s.nfresh;
    const int32_t count = *s.count;
    if (*s.abort) return;
    if (count < 0 || count > s.cap) {
        if (e == 0) {
            atomicOr(s.status, V1_STATUS_BAD_STATE);
            atomicOr(s.abort, 1u);
        }
        return;
    }
    if ((int64_t)need > (int64_t)count) {
        if (e == 0) {
            atomicOr(s.status, V1_STATUS_EXHAUSTED);
            atomicOr(s.abort, 1u);
        }
        return;
    }
    if (e >= s.n || !s.fresh[e]) return;
    const uint32_t r = s.rank[e];
    const int32_t page = s.free_stack[count - 1 - (int32_t)r];
    if (page < 0 || page >= s.cap) {  // later launches see the abort and touch nothing
        atomicOr(s.status, V1_STATUS_BAD_STATE);
        atomicOr(s.abort, 1u);
        return;
    }
    s.page_of[e] = page;
    s.fresh_list[r] = (int32_t)e;
    atomicMin(&s.class_min[s.cls[e]], page);
}

__global__ __launch_bounds__(kThreads) void pb_table(InsertState s) {
    const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= s.n || *s.abort) return;
    const int32_t c = s.cls[e];
    const int32_t page = s.fresh[e] ? s.page_of[e] : ((c & kClassLive) ? (c & ~kClassLive) : s.class_min[c]);
    s.table[e] = page;
    atomicAdd(&s.refs[page], 1);
}

// fresh pages receive the entry's bytes and key; work-groups stride over ranks
__global__ __launch_bounds__(kThreads) void pb_publish(InsertState s) {
    if (*s.abort) return;
    const uint32_t need = *s.nfresh;
    const int64_t chunks = s.page_bytes >> 4;
    for (uint32_t r = blockIdx.x; r < need; r += gridDim.x) {
        const int32_t e = s.fresh_list[r];
        const int32_t page = s.page_of[e];
        const uint4* src = reinterpret_cast<const uint4*>(s.tmp + (int64_t)e * s.page_bytes);
        uint4* dst = reinterpret_cast<uint4*>(s.pool + (int64_t)page * s.page_bytes);
        int64_t c = threadIdx.x;
        for (; c + 3 * kThreads < chunks; c += 4 * kThreads) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = src[c + u * kThreads];
#pragma unroll
            for (int u = 0; u < 4; ++u) dst[c + u * kThreads] = v[u];
        }
        for (; c < chunks; c += kThreads) dst[c] = src[c];
        if (threadIdx.x == 0) s.pool_keys[page] = s.keys[e];
    }
}

__global__ void pb_commit(InsertState s) {
    if (threadIdx.x == 0 && !*s.abort) *s.count -= (int32_t)*s.nfresh;
}

// ---------------------------------------------------------------- release
struct ReleaseState {
    const int32_t* pages;  // [n] release order
    int32_t n;
    int32_t* refs;
    int32_t* free_stack;
    int32_t* count;
    int32_t cap;
    int32_t* status;
    uint64_t* skeys;
    uint32_t* svals;
    uint64_t* okeys;
    uint32_t* ovals;
    uint32_t* head;
    uint32_t* gid;
    uint32_t* start;
    uint32_t* ngroups;
    uint32_t* dead;   // [n] by release index
    uint32_t* drank;  // [n]
    uint32_t* ndead;
    uint32_t* abort;
};

__global__ __launch_bounds__(kThreads) void rl_input(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i == 0) *s.abort = 0;
    if (i >= s.n) return;
    s.skeys[i] = (uint64_t)(uint32_t)s.pages[i];
    s.svals[i] = (uint32_t)i;
}

__global__ __launch_bounds__(kThreads) void rl_starts(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < s.n && s.head[i]) s.start[s.gid[i]] = (uint32_t)i;
}

// Sorted by page, stably: the j-th decrement of page p (j from 0) finds the
// count refs[p] - j and kills the page iff that is 1.
__global__ __launch_bounds__(kThreads) void rl_dead(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= s.n) return;
    const uint32_t page = (uint32_t)s.okeys[i];
    const int64_t j = i - s.start[group_of(s.gid, s.head, i)];
    bool bad = page >= (uint32_t)s.cap;
    const int64_t before = bad ? 0 : (int64_t)s.refs[page] - j;
    bad |= before <= 0;
    s.dead[s.ovals[i]] = before == 1 ? 1u : 0u;
    if (bad) {
        atomicOr(s.status, V1_STATUS_UNDERFLOW);
        atomicOr(s.abort, 1u);
    }
}

__global__ __launch_bounds__(kThreads) void rl_commit(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (*s.abort) return;
    const int32_t count = *s.count;
    if (count < 0 || (int64_t)count + *s.ndead > s.cap) {  // more dead pages than free slots
        if (i == 0) {
            atomicOr(s.status, V1_STATUS_BAD_STATE);
            atomicOr(s.abort, 1u);
        }
        return;
    }
    if (i >= s.n) return;
    if (s.dead[i]) s.free_stack[count + (int32_t)s.drank[i]] = s.pages[i];
    // the last decrement of each page writes its new count
    if (i + 1 == s.n || s.okeys[i + 1] != s.okeys[i]) {
        const uint32_t page = (uint32_t)s.okeys[i];
        const int64_t size = i + 1 - s.start[group_of(s.gid, s.head, i)];
        s.refs[page] -= (int32_t)size;
    }
}

__global__ void rl_count(ReleaseState s) {
    if (threadIdx.x == 0 && !*s.abort) *s.count += (int32_t)*s.ndead;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

struct Carver {
    int64_t at = 0;
    int64_t take(int64_t bytes) {
        const int64_t o = at;
        at = align256(at + std::max<int64_t>(bytes, 4));
        return o;
    }
};

struct InsertLayout {
    int64_t live_flag, live_off, nlive, skeys, svals, okeys, ovals, head, gid, start, ngroups, pos_of, cls, fresh,
        rank, nfresh, fresh_list, page_of, class_min, slow, nslow, abort, sort_ws, scan_ws, total;
};

InsertLayout insert_layout(int64_t cap, int64_t n) {
    const int64_t m = cap + n;
    Carver c;
    InsertLayout L{};
    L.live_flag = c.take(cap * 4);
    L.live_off = c.take(cap * 4);
    L.nlive = c.take(4);
    L.skeys = c.take(m * 8);
    L.svals = c.take(m * 4);
    L.okeys = c.take(m * 8);
    L.ovals = c.take(m * 4);
    L.head = c.take(m * 4);
    L.gid = c.take(m * 4);
    L.start = c.take(m * 4);
    L.ngroups = c.take(4);
    L.pos_of = c.take(n * 4);
    L.cls = c.take(n * 4);
    L.fresh = c.take(n * 4);
    L.rank = c.take(n * 4);
    L.nfresh = c.take(4);
    L.fresh_list = c.take(n * 4);
    L.page_of = c.take(n * 4);
    L.class_min = c.take(n * 4);
    L.slow = c.take(kSlowMax * 4);
    L.nslow = c.take(4);
    L.abort = c.take(4);
    L.sort_ws = c.take(sort_pairs_workspace(m));
    L.scan_ws = c.take(scan_workspace(m));
    L.total = c.at;
    return L;
}

struct ReleaseLayout {
    int64_t skeys, svals, okeys, ovals, head, gid, start, ngroups, dead, drank, ndead, abort, sort_ws, scan_ws, total;
};

ReleaseLayout release_layout(int64_t n) {
    Carver c;
    ReleaseLayout L{};
    L.skeys = c.take(n * 8);
    L.svals = c.take(n * 4);
    L.okeys = c.take(n * 8);
    L.ovals = c.take(n * 4);
    L.head = c.take(n * 4);
    L.gid = c.take(n * 4);
    L.start = c.take(n * 4);
    L.ngroups = c.take(4);
    L.dead = c.take(n * 4);
    L.drank = c.take(n * 4);
    L.ndead = c.take(4);
    L.abort = c.take(4);
    L.sort_ws = c.take(sort_pairs_workspace(n));
    L.scan_ws = c.take(scan_workspace(n));
    L.total = c.at;
    return L;
}

template <typename T>
T* at(void* w, int64_t off) {
    return reinterpret_cast<T*>(static_cast<uint8_t*>(w) + off);
}

dim3 grid_for(int64_t k) { return dim3((uint32_t)cdiv(std::max<int64_t>(k, 1), kThreads)); }

}  // namespace
}  // namespace v1

using namespace v1;

#define V1_CHECKED(name, ...)              \
    do {                                   \
        __VA_ARGS__;                       \
        const int rc_ = V1_LAUNCHED(name); \
        if (rc_ != V1_OK) return rc_;      \
    } while (0)
#define V1_OK_OR_RETURN(expr)         \
    do {                              \
        const int rc_ = (expr);       \
        if (rc_ != V1_OK) return rc_; \
    } while (0)

extern "C" int64_t v1_page_insert_workspace(int32_t capacity, int32_t n) {
    if (capacity <= 0 || n < 0) return 0;
    return insert_layout(capacity, n).total;
}

extern "C" int v1_page_insert(uint8_t* pool, int64_t* pool_keys, int32_t* refs, int32_t* free_stack, int32_t* count,
                              int32_t capacity, int64_t page_bytes, const int64_t* keys, const uint8_t* tmp,
                              const int32_t* req, int32_t n, int32_t* table, int32_t* status, void* workspace,
                              int64_t workspace_bytes, void* stream) {
    const char* name = "page_insert";
    V1_REQUIRE(capacity > 0 && capacity < kClassLive && n >= 0, "page_insert: capacity must be in (0, 2^30), n >= 0");
    V1_REQUIRE((int64_t)capacity + n < (1ll << 31) - 1, "page_insert: capacity + n must stay below 2^31 - 1");
    V1_REQUIRE(page_bytes > 0 && page_bytes % 16 == 0, "page_insert: page_bytes must be a positive multiple of 16");
    V1_REQUIRE(pool && pool_keys && refs && free_stack && count && status, "page_insert: null pool buffer");
    V1_REQUIRE(n == 0 || (keys && tmp && req && table), "page_insert: null batch buffer");
    V1_REQUIRE((reinterpret_cast<uintptr_t>(pool) & 15) == 0 && (reinterpret_cast<uintptr_t>(tmp) & 15) == 0,
               "page_insert: pages must be 16-byte aligned");
    const InsertLayout L = insert_layout(capacity, n);
    V1_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, "page_insert: workspace of %lld bytes required",
               (long long)L.total);
    if (n == 0) return V1_OK;
    void* w = workspace;
    InsertState s{pool, pool_keys, refs, free_stack, count, capacity, page_bytes, keys, tmp, req, n, table, status,
                  at<uint32_t>(w, L.live_flag), at<uint32_t>(w, L.live_off), at<uint32_t>(w, L.nlive),
                  at<uint64_t>(w, L.skeys), at<uint32_t>(w, L.svals), at<uint64_t>(w, L.okeys),
                  at<uint32_t>(w, L.ovals), at<uint32_t>(w, L.head), at<uint32_t>(w, L.gid),
                  at<uint32_t>(w, L.start), at<uint32_t>(w, L.ngroups), at<int32_t>(w, L.pos_of),
                  at<int32_t>(w, L.cls), at<uint32_t>(w, L.fresh), at<uint32_t>(w, L.rank),
                  at<uint32_t>(w, L.nfresh), at<int32_t>(w, L.fresh_list), at<int32_t>(w, L.page_of),
                  at<int32_t>(w, L.class_min), at<int32_t>(w, L.slow), at<uint32_t>(w, L.nslow),
                  at<uint32_t>(w, L.abort)};
    hipStream_t st = as_stream(stream);
    const int64_t m = (int64_t)capacity + n;
    void* scan_ws = at<uint8_t>(w, L.scan_ws);
    const int64_t scan_bytes = scan_workspace(m);
    V1_CHECKED(name, hipLaunchKernelGGL(pb_live_flags, grid_for(capacity), dim3(kThreads), 0, st, s));
    V1_OK_OR_RETURN(scan_exclusive(s.live_flag, s.live_off, s.nlive, capacity, scan_ws, scan_bytes, st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_sort_input, grid_for(std::max<int64_t>(capacity, n)), dim3(kThreads), 0,
                                        st, s));
    V1_OK_OR_RETURN(sort_pairs(s.skeys, s.svals, s.okeys, s.ovals, m, 64, at<uint8_t>(w, L.sort_ws),
                               sort_pairs_workspace(m), st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_heads, grid_for(m), dim3(kThreads), 0, st, s.okeys, s.head, m));
    V1_OK_OR_RETURN(scan_exclusive(s.head, s.gid, s.ngroups, m, scan_ws, scan_bytes, st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_groups, grid_for(m), dim3(kThreads), 0, st, s, m));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_classify, dim3((uint32_t)cdiv(n, kThreads / kWave)), dim3(kThreads), 0,
                                        st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_slow, dim3(1), dim3(kWave), 0, st, s, m));
    V1_OK_OR_RETURN(scan_exclusive(s.fresh, s.rank, s.nfresh, n, scan_ws, scan_bytes, st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_allocate, grid_for(n), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_table, grid_for(n), dim3(kThreads), 0, st, s));
    const uint32_t pub_groups = (uint32_t)std::min<int64_t>(n, 8 * (int64_t)device_cus());
    V1_CHECKED(name, hipLaunchKernelGGL(pb_publish, dim3(pub_groups), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_commit, dim3(1), dim3(kWave), 0, st, s));
    return V1_OK;
}

extern "C" int64_t v1_page_release_workspace(int32_t n) {
    if (n < 0) return 0;
    return release_layout(n).total;
}

extern "C" int v1_page_release(const int32_t* pages, int32_t n, int32_t* refs, int32_t* free_stack, int32_t* count,
                               int32_t capacity, int32_t* status, void* workspace, int64_t workspace_bytes,
                               void* stream) {
    const char* name = "page_release";
    V1_REQUIRE(capacity > 0 && n >= 0, "page_release: capacity must be positive, n >= 0");
    V1_REQUIRE(refs && free_stack && count && status && (n == 0 || pages), "page_release: null buffer");
    const ReleaseLayout L = release_layout(n);
    V1_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, "page_release: workspace of %lld bytes required",
               (long long)L.total);
    if (n == 0) return V1_OK;
    void* w = workspace;
    ReleaseState s{pages, n, refs, free_stack, count, capacity, status, at<uint64_t>(w, L.skeys),
                   at<uint32_t>(w, L.svals), at<uint64_t>(w, L.okeys), at<uint32_t>(w, L.ovals),
                   at<uint32_t>(w, L.head), at<uint32_t>(w, L.gid), at<uint32_t>(w, L.start),
                   at<uint32_t>(w, L.ngroups), at<uint32_t>(w, L.dead), at<uint32_t>(w, L.drank),
                   at<uint32_t>(w, L.ndead), at<uint32_t>(w, L.abort)};
    hipStream_t st = as_stream(stream);
    void* scan_ws = at<uint8_t>(w, L.scan_ws);
    const int64_t scan_bytes = scan_workspace(n);
    V1_CHECKED(name, hipLaunchKernelGGL(rl_input, grid_for(n), dim3(kThreads), 0, st, s));
    V1_OK_OR_RETURN(sort_pairs(s.skeys, s.svals, s.okeys, s.ovals, n, 32, at<uint8_t>(w, L.sort_ws),
                               sort_pairs_workspace(n), st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_heads, grid_for(n), dim3(kThreads), 0, st, s.okeys, s.head, n));
    V1_OK_OR_RETURN(scan_exclusive(s.head, s.gid, s.ngroups, n, scan_ws, scan_bytes, st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_starts, grid_for(n), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_dead, grid_for(n), dim3(kThreads), 0, st, s));
    V1_OK_OR_RETURN(scan_exclusive(s.dead, s.drank, s.ndead, n, scan_ws, scan_bytes, st, name));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_commit, grid_for(n), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_count, dim3(1), dim3(kWave), 0, st, s));
    return V1_OK;
}
