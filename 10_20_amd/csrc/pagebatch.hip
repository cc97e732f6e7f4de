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
// Parallel form.  An open-addressing hash table keyed by the 64-bit key holds,
// per key, the lowest live page and the first entry (atomicMin): the key's
// representative is that live page, else that entry.  An entry whose bytes
// equal its representative's resolves at once: a live representative is its
// page; otherwise the entries of the representative's request are fresh and
// later entries take the lowest of those fresh pages.  Entries whose bytes
// differ from their representative (key collisions) first look for an equal
// live page (one wave each, pages in ascending order), then one wave resolves
// the rest in request order against the earlier colliding entries.  Fresh
// ranks are one prefix sum.  A batch that would exhaust the free stack, holds
// more than kSlowMax colliding entries or has decreasing request ids changes
// nothing and reports it in the status word.
//
// Release needs no ordering pass: with c decrements of page p in the list and
// refs[p] = r, the page dies iff c == r, at its last occurrence in the list
// (c > r is an underflow).  Counts and last occurrences are per-page atomics.
// Popular keys and pages repeat across a batch and atomics on one address
// serialise, so the combining kernels first merge equal keys or pages of a
// work-group in an LDS hash table and then touch memory once per distinct one.
#include "common.h"

namespace v1 {
namespace {

constexpr uint64_t kEmpty = ~0ull;          // free hash slot; the key ~0 itself lives in slot S
constexpr int32_t kNone = 0x7fffffff;
constexpr int32_t kClassLive = 0x40000000;  // class of an entry: live page | kClassLive, else its first entry
constexpr int32_t kSlowMax = 4096;          // colliding entries resolved per batch
constexpr int kThreads = 256;
constexpr int kAggThreads = 1024;  // work-group of the combining kernels
constexpr int kAggSlots = 2048;    // their LDS hash slots (>= 2 x kAggThreads, a power of two)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
    uint64_t* hkeys;      // [S + 1]
    int32_t* hlive;       // [S + 1] lowest live page of the key
    int32_t* hfirst;      // [S + 1] first entry of the key
    uint32_t hmask;       // S - 1, S a power of two >= 2 (cap + n)
    int32_t* slot_of;     // [n]
    int32_t* cls;         // [n]
    uint32_t* fresh;      // [n]
    uint32_t* rank;       // [n]
    uint32_t* nfresh;
    int32_t* fresh_list;  // [n] rank -> entry
    int32_t* page_of;     // [n] fresh page of a fresh entry
    int32_t* class_min;   // [n] lowest fresh page of a batch class
    int32_t* slow;        // [kSlowMax] colliding entries (any order)
    int32_t* slow_live;   // [kSlowMax] their lowest equal live page, or -1
    uint32_t* nslow;
    uint32_t* abort;      // nonzero: leave the pool unchanged
};

__device__ __forceinline__ void fail(const InsertState& s, int bit) {
    atomicOr(s.status, bit);
    atomicOr(s.abort, 1u);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // SplitMix64 finaliser
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Slot of `key`, claimed if absent; -1 when the table is full (it is sized to
// stay at most half full, so this does not happen for valid calls).
__device__ int64_t hash_slot(const InsertState& s, uint64_t key) {
    if (key == kEmpty) return (int64_t)s.hmask + 1;
    uint32_t h = (uint32_t)mix64(key) & s.hmask;
    for (uint32_t probe = 0; probe <= s.hmask; ++probe) {
        const uint64_t k = __hip_atomic_load(&s.hkeys[h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (k == key) return h;
        if (k == kEmpty) {
            const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long*>(&s.hkeys[h]), kEmpty, key);
            if (old == kEmpty || old == key) return h;
        }
        h = (h + 1) & s.hmask;
    }
    return -1;
}

// LDS slot of a non-negative id in an open-addressing table of kAggSlots
// slots (-1 = free); a work-group holds at most kAggThreads ids, so a free slot
// is always found.
__device__ __forceinline__ int agg_slot(int32_t* ids, int32_t id) {
    uint32_t h = ((uint32_t)id * 0x9E3779B1u) & (kAggSlots - 1);
    for (int probe = 0; probe < kAggSlots; ++probe) {
        const int32_t old = atomicCAS(&ids[h], -1, id);
        if (old == -1 || old == id) return (int)h;
        h = (h + 1) & (kAggSlots - 1);
    }
    return -1;
}

__device__ __forceinline__ const uint8_t* entry_bytes(const InsertState& s, int64_t e) {
    return s.tmp + e * s.page_bytes;
}
__device__ __forceinline__ const uint8_t* page_bytes_at(const InsertState& s, int64_t p) {
    return s.pool + p * s.page_bytes;
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

__global__ __launch_bounds__(kThreads) void pb_init(InsertState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i <= (int64_t)s.hmask + 1) {
        s.hkeys[i] = kEmpty;
        s.hlive[i] = kNone;
        s.hfirst[i] = kNone;
    }
    if (i == 0) {
        *s.nslow = 0;
        *s.abort = 0;
    }
}

// Live pages and entries into the table, and the request order check.  The
// entries of a work-group first meet in an LDS table, so that one lane per
// distinct key probes the global table and takes the atomicMin (a popular key
// otherwise puts thousands of atomics on one address).
__global__ __launch_bounds__(kAggThreads) void pb_hash(InsertState s) {
    __shared__ uint64_t lkey[kAggSlots];
    __shared__ int32_t lslot[kAggSlots];
    __shared__ int32_t lmin[kAggSlots];
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads) {
        lkey[t] = kEmpty;
        lmin[t] = kNone;
    }
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * kAggThreads + threadIdx.x;
    if (i < s.cap && s.refs[i] > 0) {  // live pages: keys rarely repeat
        const int64_t slot = hash_slot(s, (uint64_t)s.pool_keys[i]);
        if (slot < 0) fail(s, V1_STATUS_BAD_STATE);
        else if (__hip_atomic_load(&s.hlive[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > (int32_t)i)
            atomicMin(&s.hlive[slot], (int32_t)i);
    }
    const bool entry = i < s.n;
    const uint64_t key = entry ? (uint64_t)s.keys[i] : kEmpty;
    int h = -1;
    if (entry && key != kEmpty) {
        uint32_t p = (uint32_t)mix64(key) & (kAggSlots - 1);
        for (int probe = 0; probe < kAggSlots; ++probe) {
            const uint64_t old = atomicCAS(reinterpret_cast<unsigned long long*>(&lkey[p]), kEmpty, key);
            if (old == kEmpty || old == key) {
                h = (int)p;
                break;
            }
            p = (p + 1) & (kAggSlots - 1);
        }
        if (h >= 0) atomicMin(&lmin[h], (int32_t)i);
        else fail(s, V1_STATUS_BAD_STATE);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads) {
        if (lkey[t] == kEmpty) continue;
        const int64_t g = hash_slot(s, lkey[t]);
        lslot[t] = (int32_t)g;
        if (g < 0) fail(s, V1_STATUS_BAD_STATE);
        else if (__hip_atomic_load(&s.hfirst[g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > lmin[t])
            atomicMin(&s.hfirst[g], lmin[t]);
    }
    __syncthreads();
    if (entry) {
        int64_t slot;
        if (key == kEmpty) {  // the all-ones key has its own slot
            slot = (int64_t)s.hmask + 1;
            atomicMin(&s.hfirst[slot], (int32_t)i);
        } else {
            slot = h >= 0 ? lslot[h] : -1;
        }
        s.slot_of[i] = (int32_t)slot;
        s.class_min[i] = kNone;
        if (i + 1 < s.n && s.req[i] > s.req[i + 1]) fail(s, V1_STATUS_BAD_ORDER);
    }
}

// One wave per entry: its class from the key's representative.
__global__ __launch_bounds__(kThreads) void pb_classify(InsertState s) {
    const int64_t e = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (e >= s.n || *s.abort) return;
    const int64_t slot = s.slot_of[e];
    const int32_t live = s.hlive[slot];
    const int32_t first = s.hfirst[slot];
    bool same;
    if (live != kNone) same = wave_equal(entry_bytes(s, e), page_bytes_at(s, live), s.page_bytes);
    else same = first == e || wave_equal(entry_bytes(s, e), entry_bytes(s, first), s.page_bytes);
    if (__lane_id() != 0) return;
    if (!same) {
        s.cls[e] = -1;
        s.fresh[e] = 0;
        const uint32_t k = atomicAdd(s.nslow, 1u);
        if (k < (uint32_t)kSlowMax) s.slow[k] = (int32_t)e;
    } else if (live != kNone) {
        s.cls[e] = live | kClassLive;
        s.fresh[e] = 0;
    } else {
        s.cls[e] = first;
        s.fresh[e] = s.req[e] == s.req[first] ? 1u : 0u;
    }
}

// One wave per colliding entry: the lowest live page with its key and bytes.
__global__ __launch_bounds__(kThreads) void pb_slow_live(InsertState s) {
    const uint32_t k = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    const uint32_t ns = *s.nslow;
    if (k >= ns || k >= (uint32_t)kSlowMax || *s.abort) return;
    const int32_t e = s.slow[k];
    const int64_t key = s.keys[e];
    int32_t found = -1;
    for (int32_t base = 0; base < s.cap && found < 0; base += kWave) {
        const int32_t j = base + __lane_id();
        uint64_t cand = __ballot(j < s.cap && s.refs[min(j, s.cap - 1)] > 0 && s.pool_keys[min(j, s.cap - 1)] == key);
        while (cand && found < 0) {
            const int32_t p = base + __ffsll((unsigned long long)cand) - 1;
            if (wave_equal(entry_bytes(s, e), page_bytes_at(s, p), s.page_bytes)) found = p;
            cand &= cand - 1;
        }
    }
    if (__lane_id() == 0) s.slow_live[k] = found;
}

// The colliding entries without an equal live page, one wave, in entry order:
// the class of the earliest such entry with equal key and bytes, else a class
// of its own.
__global__ __launch_bounds__(kWave) void pb_slow(InsertState s) {
    __shared__ int32_t list[kSlowMax];
    __shared__ int32_t list_live[kSlowMax];
    __shared__ int32_t list_cls[kSlowMax];
    const uint32_t ns = *s.nslow;
    if (ns == 0 || *s.abort) return;
    const int l = __lane_id();
    if (ns > (uint32_t)kSlowMax) {
        if (l == 0) fail(s, V1_STATUS_COLLISIONS);
        return;
    }
    // order by entry (distinct values): rank = number of smaller entries
    for (uint32_t k = l; k < ns; k += kWave) list_cls[k] = s.slow[k];
    __syncthreads();
    for (uint32_t k = l; k < ns; k += kWave) {
        const int32_t e = list_cls[k];
        uint32_t r = 0;
        for (uint32_t j = 0; j < ns; ++j) r += list_cls[j] < e ? 1u : 0u;
        list[r] = e;
        list_live[r] = s.slow_live[k];
    }
    __syncthreads();
    for (uint32_t k = 0; k < ns; ++k) {
        const int32_t e = list[k];
        int32_t c = list_live[k] >= 0 ? (list_live[k] | kClassLive) : -1;
        for (uint32_t k2 = 0; c < 0 && k2 < k; ++k2) {
            const int32_t y = list[k2];
            if (list_live[k2] >= 0 || s.keys[y] != s.keys[e]) continue;
            if (wave_equal(entry_bytes(s, e), entry_bytes(s, y), s.page_bytes)) c = list_cls[k2];
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
        if (e == 0) fail(s, V1_STATUS_BAD_STATE);
        return;
    }
    if ((int64_t)need > (int64_t)count) {
        if (e == 0) fail(s, V1_STATUS_EXHAUSTED);
        return;
    }
    if (e >= s.n || !s.fresh[e]) return;
    const uint32_t r = s.rank[e];
    const int32_t page = s.free_stack[count - 1 - (int32_t)r];
    if (page < 0 || page >= s.cap) {  // later launches see the abort and touch nothing
        fail(s, V1_STATUS_BAD_STATE);
        return;
    }
    s.page_of[e] = page;
    s.fresh_list[r] = (int32_t)e;
    atomicMin(&s.class_min[s.cls[e]], page);
}

// table and reference counts; the entries of a work-group add per page in LDS
// first, then once per distinct page in memory
__global__ __launch_bounds__(kAggThreads) void pb_table(InsertState s) {
    __shared__ int32_t ids[kAggSlots];
    __shared__ int32_t cnt[kAggSlots];
    if (*s.abort) return;
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads) {
        ids[t] = -1;
        cnt[t] = 0;
    }
    __syncthreads();
    const int64_t e = (int64_t)blockIdx.x * kAggThreads + threadIdx.x;
    if (e < s.n) {
        const int32_t c = s.cls[e];
        const int32_t page = s.fresh[e] ? s.page_of[e] : ((c & kClassLive) ? (c & ~kClassLive) : s.class_min[c]);
        s.table[e] = page;
        const int h = agg_slot(ids, page);
        if (h >= 0) atomicAdd(&cnt[h], 1);
        else fail(s, V1_STATUS_BAD_STATE);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads)
        if (ids[t] >= 0) atomicAdd(&s.refs[ids[t]], cnt[t]);
}

// fresh pages receive the entry's bytes and key; work-groups stride over ranks
__global__ __launch_bounds__(kThreads) void pb_publish(InsertState s) {
    if (*s.abort) return;
    const uint32_t need = *s.nfresh;
    const int64_t chunks = s.page_bytes >> 4;
    for (uint32_t r = blockIdx.x; r < need; r += gridDim.x) {
        const int32_t e = s.fresh_list[r];
        const int32_t page = s.page_of[e];
        const u32x4* src = reinterpret_cast<const u32x4*>(entry_bytes(s, e));
        u32x4* dst = reinterpret_cast<u32x4*>(s.pool + (int64_t)page * s.page_bytes);
        int64_t c = threadIdx.x;
        for (; c + 3 * kThreads < chunks; c += 4 * kThreads) {
            const u32x4 v0 = __builtin_nontemporal_load(src + c);
            const u32x4 v1 = __builtin_nontemporal_load(src + c + kThreads);
            const u32x4 v2 = __builtin_nontemporal_load(src + c + 2 * kThreads);
            const u32x4 v3 = __builtin_nontemporal_load(src + c + 3 * kThreads);
            __builtin_nontemporal_store(v0, dst + c);
            __builtin_nontemporal_store(v1, dst + c + kThreads);
            __builtin_nontemporal_store(v2, dst + c + 2 * kThreads);
            __builtin_nontemporal_store(v3, dst + c + 3 * kThreads);
        }
        for (; c < chunks; c += kThreads) __builtin_nontemporal_store(__builtin_nontemporal_load(src + c), dst + c);
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
    int32_t* cnt;      // [cap] decrements per page
    int32_t* last;     // [cap] last list index per page
    uint32_t* dead;    // [n]
    uint32_t* drank;   // [n]
    uint32_t* ndead;
    uint32_t* abort;
};

__device__ __forceinline__ void rfail(const ReleaseState& s, int bit) {
    atomicOr(s.status, bit);
    atomicOr(s.abort, 1u);
}

__global__ __launch_bounds__(kThreads) void rl_init(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < s.cap) {
        s.cnt[i] = 0;
        s.last[i] = -1;
    }
    if (i == 0) *s.abort = 0;
}

// decrements and last list index per page, combined per work-group in LDS
__global__ __launch_bounds__(kAggThreads) void rl_count(ReleaseState s) {
    __shared__ int32_t ids[kAggSlots];
    __shared__ int32_t cnt[kAggSlots];
    __shared__ int32_t last[kAggSlots];
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads) {
        ids[t] = -1;
        cnt[t] = 0;
        last[t] = -1;
    }
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * kAggThreads + threadIdx.x;
    if (i < s.n) {
        const int32_t p = s.pages[i];
        if (p >= 0 && p < s.cap) {
            const int h = agg_slot(ids, p);
            if (h >= 0) {
                atomicAdd(&cnt[h], 1);
                atomicMax(&last[h], (int32_t)i);
            } else {
                rfail(s, V1_STATUS_BAD_STATE);
            }
        } else {
            rfail(s, V1_STATUS_UNDERFLOW);
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < kAggSlots; t += kAggThreads) {
        if (ids[t] < 0) continue;
        atomicAdd(&s.cnt[ids[t]], cnt[t]);
        atomicMax(&s.last[ids[t]], last[t]);
    }
}

__global__ __launch_bounds__(kThreads) void rl_dead(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= s.n) return;
    const int32_t p = s.pages[i];
    uint32_t d = 0;
    if (p >= 0 && p < s.cap) {
        const int32_t c = s.cnt[p], r = s.refs[p];
        if (c > r) rfail(s, V1_STATUS_UNDERFLOW);
        d = (c == r && s.last[p] == i) ? 1u : 0u;
    }
    s.dead[i] = d;
}

__global__ __launch_bounds__(kThreads) void rl_commit(ReleaseState s) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (*s.abort) return;
    const int32_t count = *s.count;
    if (count < 0 || (int64_t)count + *s.ndead > s.cap) {  // more dead pages than free slots
        if (i == 0) rfail(s, V1_STATUS_BAD_STATE);
        return;
    }
    if (i >= s.n) return;
    const int32_t p = s.pages[i];
    if (s.dead[i]) s.free_stack[count + (int32_t)s.drank[i]] = p;
    if (s.last[p] == i) s.refs[p] -= s.cnt[p];
}

__global__ void rl_finish(ReleaseState s) {
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

int64_t hash_size(int64_t cap, int64_t n) {
    int64_t S = 1024;
    while (S < 2 * (cap + n)) S <<= 1;
    return S;
}

struct InsertLayout {
    int64_t S, hkeys, hlive, hfirst, slot_of, cls, fresh, rank, nfresh, fresh_list, page_of, class_min, slow,
        slow_live, nslow, abort, scan_ws, total;
};

InsertLayout insert_layout(int64_t cap, int64_t n) {
    Carver c;
    InsertLayout L{};
    L.S = hash_size(cap, n);
    L.hkeys = c.take((L.S + 1) * 8);
    L.hlive = c.take((L.S + 1) * 4);
    L.hfirst = c.take((L.S + 1) * 4);
    L.slot_of = c.take(n * 4);
    L.cls = c.take(n * 4);
    L.fresh = c.take(n * 4);
    L.rank = c.take(n * 4);
    L.nfresh = c.take(4);
    L.fresh_list = c.take(n * 4);
    L.page_of = c.take(n * 4);
    L.class_min = c.take(n * 4);
    L.slow = c.take(kSlowMax * 4);
    L.slow_live = c.take(kSlowMax * 4);
    L.nslow = c.take(4);
    L.abort = c.take(4);
    L.scan_ws = c.take(scan_workspace(n));
    L.total = c.at;
    return L;
}

struct ReleaseLayout {
    int64_t cnt, last, dead, drank, ndead, abort, scan_ws, total;
};

ReleaseLayout release_layout(int64_t cap, int64_t n) {
    Carver c;
    ReleaseLayout L{};
    L.cnt = c.take(cap * 4);
    L.last = c.take(cap * 4);
    L.dead = c.take(n * 4);
    L.drank = c.take(n * 4);
    L.ndead = c.take(4);
    L.abort = c.take(4);
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
    V1_REQUIRE((int64_t)capacity + n < (1ll << 29), "page_insert: capacity + n must stay below 2^29");
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
                  at<uint64_t>(w, L.hkeys), at<int32_t>(w, L.hlive), at<int32_t>(w, L.hfirst),
                  (uint32_t)(L.S - 1), at<int32_t>(w, L.slot_of), at<int32_t>(w, L.cls), at<uint32_t>(w, L.fresh),
                  at<uint32_t>(w, L.rank), at<uint32_t>(w, L.nfresh), at<int32_t>(w, L.fresh_list),
                  at<int32_t>(w, L.page_of), at<int32_t>(w, L.class_min), at<int32_t>(w, L.slow),
                  at<int32_t>(w, L.slow_live), at<uint32_t>(w, L.nslow), at<uint32_t>(w, L.abort)};
    hipStream_t st = as_stream(stream);
    V1_CHECKED(name, hipLaunchKernelGGL(pb_init, grid_for(L.S + 1), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_hash, dim3((uint32_t)cdiv(std::max<int64_t>(capacity, n), kAggThreads)),
                                        dim3(kAggThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_classify, dim3((uint32_t)cdiv(n, kThreads / kWave)), dim3(kThreads), 0,
                                        st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_slow_live, dim3(kSlowMax / (kThreads / kWave)), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_slow, dim3(1), dim3(kWave), 0, st, s));
    V1_OK_OR_RETURN(scan_exclusive(s.fresh, s.rank, s.nfresh, n, at<uint8_t>(w, L.scan_ws), scan_workspace(n), st,
                                   name));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_allocate, grid_for(n), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_table, dim3((uint32_t)cdiv(n, kAggThreads)), dim3(kAggThreads), 0, st, s));
    const uint32_t pub_groups = (uint32_t)std::min<int64_t>(n, 8 * (int64_t)device_cus());
    V1_CHECKED(name, hipLaunchKernelGGL(pb_publish, dim3(pub_groups), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(pb_commit, dim3(1), dim3(kWave), 0, st, s));
    return V1_OK;
}

extern "C" int64_t v1_page_release_workspace(int32_t capacity, int32_t n) {
    if (capacity <= 0 || n < 0) return 0;
    return release_layout(capacity, n).total;
}

extern "C" int v1_page_release(const int32_t* pages, int32_t n, int32_t* refs, int32_t* free_stack, int32_t* count,
                               int32_t capacity, int32_t* status, void* workspace, int64_t workspace_bytes,
                               void* stream) {
    const char* name = "page_release";
    V1_REQUIRE(capacity > 0 && n >= 0, "page_release: capacity must be positive, n >= 0");
    V1_REQUIRE(refs && free_stack && count && status && (n == 0 || pages), "page_release: null buffer");
    const ReleaseLayout L = release_layout(capacity, n);
    V1_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, "page_release: workspace of %lld bytes required",
               (long long)L.total);
    if (n == 0) return V1_OK;
    void* w = workspace;
    ReleaseState s{pages, n, refs, free_stack, count, capacity, status, at<int32_t>(w, L.cnt),
                   at<int32_t>(w, L.last), at<uint32_t>(w, L.dead), at<uint32_t>(w, L.drank),
                   at<uint32_t>(w, L.ndead), at<uint32_t>(w, L.abort)};
    hipStream_t st = as_stream(stream);
    V1_CHECKED(name, hipLaunchKernelGGL(rl_init, grid_for(capacity), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_count, dim3((uint32_t)cdiv(n, kAggThreads)), dim3(kAggThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_dead, grid_for(n), dim3(kThreads), 0, st, s));
    V1_OK_OR_RETURN(scan_exclusive(s.dead, s.drank, s.ndead, n, at<uint8_t>(w, L.scan_ws), scan_workspace(n), st,
                                   name));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_commit, grid_for(n), dim3(kThreads), 0, st, s));
    V1_CHECKED(name, hipLaunchKernelGGL(rl_finish, dim3(1), dim3(kWave), 0, st, s));
    return V1_OK;
}
