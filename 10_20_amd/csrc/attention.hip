// Decode attention over the gathered workspace: the consumer that follows the
// slot gather (sglang/srt/layers/attention/v1_native/backend.py:306-315 calls
// flash_attn_with_kvcache(q[:, None], kg, vg, causal=False,
// softmax_scale=scaling) on the GatherWorkspace rows).  One query position
// per batch row, Hq query heads sharing each of Hkv KV heads (GQA group
// G = Hq / Hkv <= 4, the reference's group of 4), head dim 128, bf16 in, fp32 math, bf16 out:
//   O[b, h] = sum_j p_j v[b, j, h / G],  p = softmax_j(scale * q[b, h] . k[b, j, h / G])
// over the row's first n_b keys (n_b = seqlens[b] clamped to [0, S], or S);
// a row with no keys gives zeros.
//
// One 256-thread work-group per (KV head, row): 16 groups of 16 lanes, lane c
// holding dims 8c .. 8c+7, group g taking keys g, g+16, ...; a wave's four
// groups read four consecutive 256-byte key rows (1 KiB per load).  Pass 1
// writes scale * q . k per (head, key) to LDS and the block maximum per head;
// pass 2 streams V with p = exp(s - max) and sums p * v in registers; the 16
// groups' partial sums are added in LDS.  K and V are each read once: the
// kernel is bound by HBM (4 * G flops per key byte).
//
// Slot form: keys come straight from the K / V pools of one KV head through
// the row's slot ids (req[ids[b, j]], the GatherWorkspace mapping of
// sglang/srt/layers/attention/v1_native/kernels.py:62-77); an id below zero
// or past req, or a slot outside the pool, is a zero key and value, exactly
// what the gather writes.  Same arithmetic, without the workspace round trip;
// the row's slots are resolved into LDS first (all keys at once), so the key
// and value loads do not wait on the id -> slot chain.
#include <algorithm>

#include "common.h"

namespace v1 {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnDim = 128;
constexpr int kMaxGroup = 4;       // partial sums of 16 groups: 32 KiB of LDS
constexpr int kMaxScores = 12288;  // S * G scores in LDS (48 KiB)

// Lane p ^ J within 16-lane rows, every lane active.
template <int J>
__device__ __forceinline__ float row_xor(float v) {
    const int x = __float_as_int(v);
    if constexpr (J == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    else if constexpr (J == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    else if constexpr (J == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(x, (J << 10) | 0x1F));
}

__device__ __forceinline__ float row_sum16(float v) {
    v += row_xor<8>(v);
    v += row_xor<4>(v);
    v += row_xor<2>(v);
    v += row_xor<1>(v);
    return v;
}

// 8 bf16 (16 bytes) -> fp32, exact.
__device__ __forceinline__ void bf16x8(const uint4 w, float (&f)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(u[i] << 16);
        f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
}

// fp32 -> bf16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t to_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

struct AttnParams {
    const uint16_t* q;
    int64_t q_batch, q_head;
    const uint16_t* k;
    int64_t k_batch, k_token, k_head;
    const uint16_t* v;
    int64_t v_batch, v_token, v_head;
    const int32_t* seqlens;
    uint16_t* out;
    int64_t o_batch, o_head;
    int32_t keys;
    float scale;
    // slot form
    const int32_t* ids;
    int64_t ids_stride;
    const int32_t* req;
    int64_t req_len;
    int64_t pool_rows;
};

// Floats of LDS before the slot rows: the scores [G][keys], later reused for
// the partial sums [16][G][128] and their weights [16][G].
template <int G>
__host__ __device__ constexpr int64_t attn_floats(int64_t keys) {
    return G * keys > 16 * G * kAttnDim + 16 * G ? G * keys : 16 * G * kAttnDim + 16 * G;
}

template <int G, bool SLOTS>
__global__ __launch_bounds__(kAttnThreads) void decode_attn_kernel(AttnParams p) {
    extern __shared__ float smem[];  // scores [G][keys], later partials [16][G][128] + sums [16][G]
    __shared__ float red[16][kMaxGroup];
    const int64_t b = blockIdx.y;
    const int32_t kvh = blockIdx.x;
    const int32_t t = threadIdx.x, g = t >> 4, c = t & 15;
    const int32_t S = p.keys;
    const int32_t n = p.seqlens ? min(max(p.seqlens[b], 0), S) : S;

    float qf[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint4 w = *reinterpret_cast<const uint4*>(p.q + b * p.q_batch + (int64_t)(kvh * G + h) * p.q_head + 8 * c);
        bf16x8(w, qf[h]);
    }
    const uint16_t* kr = p.k + (SLOTS ? 0 : b * p.k_batch) + (int64_t)kvh * p.k_head + 8 * c;
    const uint16_t* vr = p.v + (SLOTS ? 0 : b * p.v_batch) + (int64_t)kvh * p.v_head + 8 * c;
    // slot form: every key's pool row (-1: a zero key) into LDS past the scores / partials
    int32_t* rows_s = reinterpret_cast<int32_t*>(smem + attn_floats<G>(S));
    if constexpr (SLOTS) {
        for (int32_t j = t; j < n; j += kAttnThreads) {
            const int32_t id = p.ids[b * p.ids_stride + j];
            int32_t slot = -1;
            if (id >= 0 && id < p.req_len) {
                slot = p.req[id];
                if (slot < 0 || slot >= p.pool_rows) slot = -1;
            }
            rows_s[j] = slot;
        }
        __syncthreads();
    }
    // row of key j in the K / V arrays (-1: a zero key)
    auto key_row = [&](int32_t j) __attribute__((always_inline)) -> int64_t {
        if constexpr (!SLOTS) return j;
        else return rows_s[j];
    };

    // pass 1: scores and the group maxima
    float mx[G];
#pragma unroll
    for (int h = 0; h < G; ++h) mx[h] = -__builtin_inff();
    for (int32_t j0 = g; j0 < n; j0 += 64) {
        uint4 kw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int32_t j = j0 + 16 * u;
            const int64_t r = j < n ? key_row(j) : -1;
            kw[u] = r >= 0 ? *reinterpret_cast<const uint4*>(kr + r * p.k_token) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int32_t j = j0 + 16 * u;
            float kf[8];
            bf16x8(kw[u], kf);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float part = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) part = fmaf(qf[h][i], kf[i], part);
                const float s = row_sum16(part) * p.scale;
                if (j < n) {
                    if (c == h) smem[h * S + j] = s;
                    mx[h] = fmaxf(mx[h], s);
                }
            }
        }
    }
    if (c == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) red[g][h] = mx[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float m = red[0][h];
#pragma unroll
        for (int k = 1; k < 16; ++k) m = fmaxf(m, red[k][h]);
        mx[h] = m;
    }

    // pass 2: exp-weighted sums of V
    float acc[G][8], sum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        sum[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
    }
    for (int32_t j0 = g; j0 < n; j0 += 64) {
        uint4 vw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int32_t j = j0 + 16 * u;
            const int64_t r = j < n ? key_row(j) : -1;
            vw[u] = r >= 0 ? *reinterpret_cast<const uint4*>(vr + r * p.v_token) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int32_t j = j0 + 16 * u;
            if (j >= n) continue;
            float vf[8];
            bf16x8(vw[u], vf);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float e = __expf(smem[h * S + j] - mx[h]);
                sum[h] += e;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(e, vf[i], acc[h][i]);
            }
        }
    }
    __syncthreads();  // the scores are no longer read
    float* part = smem;                        // [16][G][128]
    float* sums = smem + 16 * G * kAttnDim;    // [16][G]
#pragma unroll
    for (int h = 0; h < G; ++h) {
        *reinterpret_cast<float4*>(part + (g * G + h) * kAttnDim + 8 * c) =
            make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        *reinterpret_cast<float4*>(part + (g * G + h) * kAttnDim + 8 * c + 4) =
            make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        if (c == 0) sums[g * G + h] = sum[h];
    }
    __syncthreads();
    for (int idx = t; idx < G * kAttnDim; idx += kAttnThreads) {
        const int h = idx / kAttnDim, d = idx % kAttnDim;
        float o = 0.f, s = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            o += part[(k * G + h) * kAttnDim + d];
            s += sums[k * G + h];
        }
        p.out[b * p.o_batch + (int64_t)(kvh * G + h) * p.o_head + d] = to_bf16(n > 0 ? o / s : 0.f);
    }
}

template <int G, bool SLOTS>
int launch_attn(const AttnParams& p, int32_t batch, int32_t heads_kv, hipStream_t st) {
    const size_t lds = sizeof(float) * (size_t)(attn_floats<G>(p.keys) + (SLOTS ? p.keys : 0));
    hipLaunchKernelGGL((decode_attn_kernel<G, SLOTS>), dim3((uint32_t)heads_kv, (uint32_t)batch), dim3(kAttnThreads),
                       lds, st, p);
    return V1_LAUNCHED("decode_attention");
}

template <bool SLOTS>
int launch_group(int32_t G, const AttnParams& p, int32_t batch, int32_t heads_kv, hipStream_t st) {
    switch (G) {
        case 1: return launch_attn<1, SLOTS>(p, batch, heads_kv, st);
        case 2: return launch_attn<2, SLOTS>(p, batch, heads_kv, st);
        case 3: return launch_attn<3, SLOTS>(p, batch, heads_kv, st);
        default: return launch_attn<4, SLOTS>(p, batch, heads_kv, st);
    }
}

}  // namespace
}  // namespace v1

using namespace v1;

extern "C" int v1_decode_attention(const void* q, int64_t q_batch, int64_t q_head, const void* k, int64_t k_batch,
                                   int64_t k_token, int64_t k_head, const void* v, int64_t v_batch, int64_t v_token,
                                   int64_t v_head, const int32_t* seqlens, void* out, int64_t o_batch, int64_t o_head,
                                   int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t keys, float scale,
                                   void* stream) {
    V1_REQUIRE(batch >= 0 && heads_kv > 0 && heads_q > 0 && heads_q % heads_kv == 0 && keys >= 0,
               "decode_attention: bad shape");
    const int32_t G = heads_q / heads_kv;
    V1_REQUIRE(G <= kMaxGroup, "decode_attention: at most %d query heads per KV head", kMaxGroup);
    V1_REQUIRE((int64_t)G * keys <= kMaxScores, "decode_attention: keys x group above %d", kMaxScores);
    const int64_t strides[] = {q_batch, q_head, k_batch, k_token, k_head, v_batch, v_token, v_head, o_batch, o_head};
    bool aligned = (reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16 == 0;
    for (int64_t s : strides) aligned = aligned && s % 8 == 0;
    V1_REQUIRE(aligned, "decode_attention: q, k, v must be 16-byte aligned with strides in multiples of 8 elements");
    if (batch == 0) return V1_OK;
    AttnParams p{static_cast<const uint16_t*>(q), q_batch, q_head, static_cast<const uint16_t*>(k), k_batch, k_token,
                 k_head, static_cast<const uint16_t*>(v), v_batch, v_token, v_head, seqlens,
                 static_cast<uint16_t*>(out), o_batch, o_head, keys, scale, nullptr, 0, nullptr, 0, 0};
    return launch_group<false>(G, p, batch, heads_kv, as_stream(stream));
}

extern "C" int v1_decode_attention_slots(const void* q, int64_t q_batch, int64_t q_head, const void* k_pool,
                                         int64_t k_slot, int64_t k_head, const void* v_pool, int64_t v_slot,
                                         int64_t v_head, int64_t pool_slots, int32_t head, const int32_t* req,
                                         int64_t req_len, const int32_t* ids, int64_t ids_stride, void* out,
                                         int64_t o_batch, int64_t o_head, int32_t rows, int32_t heads_q, int32_t keys,
                                         float scale, void* stream) {
    V1_REQUIRE(rows >= 0 && heads_q > 0 && heads_q <= kMaxGroup && keys >= 0 && head >= 0 && pool_slots >= 0,
               "decode_attention_slots: bad shape (at most %d query heads)", kMaxGroup);
    V1_REQUIRE((int64_t)heads_q * keys + keys <= kMaxScores, "decode_attention_slots: keys x (heads + 1) above %d",
               kMaxScores);
    V1_REQUIRE(req != nullptr && req_len > 0 && ids != nullptr, "decode_attention_slots: empty slot map");
    const int64_t strides[] = {q_batch, q_head, k_slot, k_head, v_slot, v_head, o_batch, o_head};
    bool aligned = (reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) |
                    reinterpret_cast<uintptr_t>(v_pool)) % 16 == 0;
    for (int64_t s : strides) aligned = aligned && s % 8 == 0;
    V1_REQUIRE(aligned, "decode_attention_slots: q and the pools must be 16-byte aligned, strides multiples of 8");
    if (rows == 0) return V1_OK;
    // the chosen KV head becomes head 0 of a one-head problem
    AttnParams p{static_cast<const uint16_t*>(q), q_batch, q_head,
                 static_cast<const uint16_t*>(k_pool) + (int64_t)head * k_head, 0, k_slot, 0,
                 static_cast<const uint16_t*>(v_pool) + (int64_t)head * v_head, 0, v_slot, 0, nullptr,
                 static_cast<uint16_t*>(out), o_batch, o_head, keys, scale, ids, ids_stride, req, req_len, pool_slots};
    return launch_group<true>(heads_q, p, rows, 1, as_stream(stream));
}
