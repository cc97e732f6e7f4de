"""Deterministic synthetic inputs for the query-indexing workloads (host numpy,
PCG64 seeded; identical on every machine).

FP8 is OCP e4m3fn.  Quantisation follows the reference rule
s = 2^ceil(log2(max(absmax, 1e-4) / 448)), x8 = e4m3(x / s)
(sglang/srt/layers/attention/v1_native/grouping.py:41-45), with the exponent
taken exactly from frexp rather than from a floating log2.

Native page layout (8448 bytes): 64 tokens x 128 FP8 bytes, then 64 fp32
scales (sglang/srt/layers/attention/v1_deepseek/kernels.py:1-3).
"""
from dataclasses import dataclass, field

import numpy as np

PAGE = 64
DIM = 128
PAGE_BYTES = 8448
MLA_ROW_BYTES = 656  # 512 FP8 latent + 64 bf16 RoPE + fp32 scales (41 x 16 B)
TOPK = 2048


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ------------------------------------------------------------------- FP8
def _e4m3_positive_values():
    """Values of the 127 non-negative finite e4m3fn codes 0x00..0x7e, ascending."""
    codes = np.arange(127)
    e = codes >> 3
    m = codes & 7
    return np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))


_E4M3_POS = _e4m3_positive_values()


def e4m3_encode(x):
    """Round-to-nearest-even float -> e4m3fn byte; |x| must be <= 448."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    if a.size and float(a.max()) > 448.0:
        raise ValueError("e4m3_encode: value beyond the e4m3fn range")
    hi = np.clip(np.searchsorted(_E4M3_POS, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dl = a - _E4M3_POS[lo]
    dh = _E4M3_POS[hi] - a
    pick_hi = (dh < dl) | ((dh == dl) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return code | (np.signbit(x).astype(np.uint8) << 7)


def pow2_scale(absmax):
    """2^ceil(log2(max(absmax, 1e-4) / 448)) in float32, exactly."""
    v = np.maximum(np.asarray(absmax, dtype=np.float32), np.float32(1e-4)) / np.float32(448.0)
    m, e = np.frexp(v)
    e = np.where(m == 0.5, e - 1, e)
    return np.ldexp(np.float32(1.0), e).astype(np.float32)


def e4m3_encode_fast(x):
    """e4m3_encode through torch's round-to-nearest-even cast (identical codes,
    checked against e4m3_encode in the tests), for large arrays."""
    import torch
    x = np.ascontiguousarray(x, dtype=np.float32)
    return torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def quantize_rows(x):
    """Per-row (token) FP8 quantisation: returns (bytes [n, d], scale [n])."""
    x = np.asarray(x, dtype=np.float32)
    s = pow2_scale(np.abs(x).max(axis=-1))
    return e4m3_encode_fast(x / s[..., None]), s


def pack_pages(k8, ks, n_pages=None):
    """Native pages [n_pages, 8448] from token keys k8 [n, 128] and scales [n]."""
    n = k8.shape[0]
    pages = n_pages if n_pages is not None else -(-n // PAGE)
    out = np.zeros((pages, PAGE_BYTES), dtype=np.uint8)
    kk = np.zeros((pages * PAGE, DIM), dtype=np.uint8)
    kk[:n] = k8
    ss = np.zeros(pages * PAGE, dtype=np.float32)
    ss[:n] = ks
    out[:, :8192] = kk.reshape(pages, 8192)
    out[:, 8192:] = ss.reshape(pages, PAGE).view(np.uint8)
    return out


def scatter_pages(pool_pages, logical_pages, table):
    """Places logical page i at physical page table[i] of a zero pool."""
    pool = np.zeros((pool_pages, logical_pages.shape[1]), dtype=np.uint8)
    pool[table[: len(logical_pages)]] = logical_pages
    return pool


# --------------------------------------------------------------- configs
@dataclass
class Workload:
    name: str
    seed: int
    arrays: dict = field(default_factory=dict)
    params: dict = field(default_factory=dict)


def config1(seed=19, rows=1024):
    """The reference example shape with FP8 N(0,1) data
    (sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:11-41):
    1024 queries x 1 head, 4097 keys in four built 1K buckets (members reversed
    per bucket), route of 40 of 64 pages (P=128), 2688 fine candidates
    (40 pages + 64 sink + 64 tail), query i sees candidates < 1664+i, Top-2048,
    native table = random pages of a 4096-page pool, 656-byte row gather."""
    g = rng(seed)
    B, P, CAP, TAKE, N, WINDOW, SINK = rows, 128, 128, 40, 4097, 64, 64
    POOL = 4096
    nt_row = g.permutation(POOL)[:P].astype(np.int32)
    rt_row = g.permutation(CAP).astype(np.int32)
    q8, qs = quantize_rows(g.standard_normal((B, DIM), dtype=np.float32))
    k8, ks = quantize_rows(g.standard_normal((N, DIM), dtype=np.float32))
    # native pool: logical page i of the request at physical page nt_row[i]
    native = scatter_pages(POOL, pack_pages(k8, ks), nt_row)
    logical_order = np.arange(4096, dtype=np.int32).reshape(4, 1024)[:, ::-1].reshape(64, 64).copy()
    members = np.full((CAP, 64), -1, dtype=np.int32)
    members[rt_row[:64]] = logical_order
    # fine pool: reordered pages at rt_row[i], then 68 tail scratch pages
    fine = np.zeros((CAP + 68, PAGE_BYTES), dtype=np.uint8)
    ro_k8, ro_ks = k8[logical_order.reshape(-1)], ks[logical_order.reshape(-1)]
    fine[rt_row[:64]] = pack_pages(ro_k8, ro_ks)
    # centers: mean of 8 consecutive reordered members, FP8 with pow2 scale
    kf = ro_k8.astype(np.int64)
    dq = decode_table()[ro_k8] * ro_ks[:, None]
    mean = dq.reshape(512, 8, DIM).sum(axis=1, dtype=np.float32) / np.float32(8.0)
    c8, cs = quantize_rows(mean)
    centers = pack_pages(c8, cs)  # 8 pages = 512 centers
    w = qs[:, None].astype(np.float32)  # H = 1: weight = q scale
    fine_lens = np.minimum(2688, 1664 + np.arange(B)).astype(np.int32)
    lat_pool = g.integers(0, 256, size=(POOL * PAGE, MLA_ROW_BYTES), dtype=np.uint8)
    del kf
    return Workload("config1", seed, dict(
        q8=q8.reshape(B, 1, DIM), w=w, native=native, fine=fine, members=members, centers=centers,
        nt=np.broadcast_to(nt_row, (B, P)).copy(), rt=np.broadcast_to(rt_row, (B, P)).copy(),
        center_table=np.arange(8, dtype=np.int32), lens=np.full(B, N, np.int32),
        takes=np.full(B, TAKE, np.int32), tail_rows=np.zeros(B, np.int32), fine_lens=fine_lens,
        latent=lat_pool),
        dict(B=B, P=P, CAP=CAP, TAKE=TAKE, N=N, WINDOW=WINDOW, SINK=SINK, TOPK=TOPK, H=1, FT_COLS=TAKE + 68,
             WIDTH=2688))


def config9(seed=9, rows=1024, heads=64, buckets=64, bucket_tokens=1024, page_fraction=0.5, sink=64,
            window=2048, route_pages=2048, pool_pages=4096):
    """The reference's published whole-query shape (coarse score + route +
    fine score + fused Top-K + x4 at 1024 queries and 64K context,
    sglang/srt/layers/attention/v1_deepseek/README.txt:117) with synthetic FP8
    N(0,1) keys and the runtime's default geometry (runtime.py:24-28, 75:
    page_fraction 0.5, sink 64, window 2048): 1024 queries x 64 heads with
    U(0,1) weights, 65536 keys in 64 built 1K buckets (members reversed per
    bucket) plus one unbuilt token, coarse scores over the 8192 centers (8 per
    built page), route of 512 of the 1024 built pages, 512 x 64 + 64 + 2048 =
    34880 fine candidates (query i sees the first 34880 - 1023 + i), Top-2048,
    native table = random pages of a 4096-page pool, 656-byte row gather."""
    g = rng(seed)
    B, PG = rows, route_pages
    NB = buckets * bucket_tokens
    N = NB + 1
    built = NB // PAGE
    TAKE = max(-(-built * int(page_fraction * 1000) // 1000), -(-TOPK // PAGE))
    CAP = PG
    nt_row = g.permutation(pool_pages)[:PG].astype(np.int32)
    rt_row = g.permutation(CAP).astype(np.int32)
    q8, _ = quantize_rows(g.standard_normal((B * heads, DIM), dtype=np.float32))
    w = g.random((B, heads), dtype=np.float32)
    k8, ks = quantize_rows(g.standard_normal((N, DIM), dtype=np.float32))
    native = scatter_pages(pool_pages, pack_pages(k8, ks), nt_row)
    logical_order = np.arange(NB, dtype=np.int32).reshape(buckets, bucket_tokens)[:, ::-1].reshape(built, PAGE).copy()
    members = np.full((CAP, PAGE), -1, dtype=np.int32)
    members[rt_row[:built]] = logical_order
    fine = np.zeros((CAP + 68, PAGE_BYTES), dtype=np.uint8)
    ro_k8, ro_ks = k8[logical_order.reshape(-1)], ks[logical_order.reshape(-1)]
    fine[rt_row[:built]] = pack_pages(ro_k8, ro_ks)
    dq = decode_table()[ro_k8] * ro_ks[:, None]
    mean = dq.reshape(NB // 8, 8, DIM).sum(axis=1, dtype=np.float32) / np.float32(8.0)
    del dq
    c8, cs = quantize_rows(mean)
    centers = pack_pages(c8, cs)
    WIDTH = TAKE * PAGE + sink + window
    fine_lens = np.minimum(WIDTH, WIDTH - (B - 1) + np.arange(B)).astype(np.int32)
    lat_pool = g.integers(0, 256, size=(pool_pages * PAGE, MLA_ROW_BYTES), dtype=np.uint8)
    return Workload("config9", seed, dict(
        q8=q8.reshape(B, heads, DIM), w=w, native=native, fine=fine, members=members, centers=centers,
        nt=np.broadcast_to(nt_row, (B, PG)).copy(), rt=np.broadcast_to(rt_row, (B, PG)).copy(),
        center_table=np.arange(centers.shape[0], dtype=np.int32), lens=np.full(B, N, np.int32),
        takes=np.full(B, TAKE, np.int32), tail_rows=np.zeros(B, np.int32), fine_lens=fine_lens,
        latent=lat_pool),
        dict(B=B, P=PG, CAP=CAP, TAKE=TAKE, N=N, WINDOW=window, SINK=sink, TOPK=TOPK, H=heads, FT_COLS=TAKE + 68,
             WIDTH=WIDTH, CENTERS=NB // 8, BUILT=built))


def splitmix64(x):
    """SplitMix64 finaliser (Steele, Lea, Flood 2014) of uint64 values."""
    z = np.asarray(x, dtype=np.uint64) + np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def config2(seed=2, requests=4096, max_pages=64, capacity=65536, zipf=1.1, collide=0, release_frac=0.5):
    """Page management: `requests` requests of U{1..max_pages} pages; each page
    is a Zipf(zipf) draw d (many pages shared), its key splitmix64(d) as int64
    and its bytes a function of d (config2_payload).  `collide` rarely-drawn
    pages get the key of another draw (equal key, other bytes).  `released`
    marks a seeded `release_frac` of the requests whose pages are released
    after the insert (config2_release_list).  Pages hold 64 MLA rows of 656
    bytes (41984 B)."""
    g = rng(seed)
    lens = g.integers(1, max_pages + 1, requests)
    n = int(lens.sum())
    draws = g.zipf(zipf, n).astype(np.uint64)
    uniq, inv, counts = np.unique(draws, return_inverse=True, return_counts=True)
    ukeys = splitmix64(uniq).view(np.int64)
    if collide:
        rare = np.flatnonzero(counts <= 3)
        victims = g.choice(rare, collide, replace=False)
        donors = g.choice(len(uniq), collide)
        donors = np.where(donors == victims, (donors + 1) % len(uniq), donors)
        ukeys = ukeys.copy()
        ukeys[victims] = ukeys[donors]
    req = np.repeat(np.arange(requests, dtype=np.int32), lens)
    released = g.random(requests) < release_frac
    return Workload("config2", seed, dict(lens=lens.astype(np.int32), req=req, draw=inv.astype(np.int32),
                                          keys=ukeys[inv], ukeys=ukeys, released=released),
                    dict(requests=requests, entries=n, distinct=len(uniq), capacity=capacity,
                         page_bytes=PAGE * MLA_ROW_BYTES))


def config2_payload(wl, page_bytes):
    """uint8 [distinct, page_bytes]: the bytes of each distinct draw (seeded)."""
    return rng(wl.seed + 1000).integers(0, 256, size=(wl.params["distinct"], page_bytes), dtype=np.uint8)


def config2_release_list(wl, table):
    """Pages of the released requests, in request order."""
    sel = wl.arrays["released"][wl.arrays["req"]]
    return np.asarray(table)[sel].astype(np.int32)


def config2_tails(wl, table, seed_offset=7):
    """Tail staging inputs of the page-management workload: request pairs
    (2k, 2k+1) share one tail (tail_rows[2k+1] = 2k), each request's native
    table lists its own pages (cycled), and its length n = 1024 j + 64 tokens
    (j in 1..3) gives a 128-token tail (64 sink + 64 tail slots, two pages)."""
    g = rng(wl.seed + seed_offset)
    lens_p = wl.arrays["lens"]
    R = len(lens_p)
    starts = np.concatenate([[0], np.cumsum(lens_p)[:-1]])
    n = np.repeat(1024 * g.integers(1, 4, (R + 1) // 2) + 64, 2)[:R].astype(np.int32)
    np_ = int(-(-int(n.max()) // PAGE))
    cols = np.arange(np_)
    nt = np.asarray(table)[starts[:, None] + cols[None, :] % lens_p[:, None]].astype(np.int32)
    tail_rows = (np.arange(R) // 2 * 2).astype(np.int32)
    return dict(nt=nt, lens=n, tail_rows=tail_rows, np=np_, scratch=2)


def config3(seed=3, rows=1024, pool_tokens=1 << 20, window_pages=512, pad=0.05):
    """K/V slot gather: 656-byte rows of a 1M-token paged pool; each query has
    its own 512-page request window (random pages of the pool) and 2048 ids
    uniform over the window's 32768 tokens, 5% set to -1."""
    g = rng(seed)
    pool_pages = pool_tokens // PAGE
    pool = g.integers(0, 256, size=(pool_tokens, MLA_ROW_BYTES), dtype=np.uint8)
    table = np.stack([g.choice(pool_pages, window_pages, replace=False) for _ in range(rows)]).astype(np.int32)
    ids = g.integers(0, window_pages * PAGE, size=(rows, TOPK), dtype=np.int64).astype(np.int32)
    ids[g.random((rows, TOPK)) < pad] = -1
    return Workload("config3", seed, dict(pool=pool, table=table, ids=ids),
                    dict(rows=rows, top=TOPK, row_bytes=MLA_ROW_BYTES, page_bits=6))


def config4(seed=4, rows=4096, ctx_tokens=32768, heads=64, first_pos=28672):
    """DeepSeek-V3.2-style prefill indexer chunk: 4096 queries x 64 heads FP8,
    32768 context keys FP8 in 64-token pages (random 512-page table), weights
    U(0,1); query i at position first_pos+i sees keys <= first_pos+i; Top-2048,
    slot mapping through the page table, 656-byte latent row gather."""
    g = rng(seed)
    pages = ctx_tokens // PAGE
    q8, _ = quantize_rows(g.standard_normal((rows * heads, DIM), dtype=np.float32))
    w = g.random((rows, heads), dtype=np.float32)
    k8, ks = quantize_rows(g.standard_normal((ctx_tokens, DIM), dtype=np.float32))
    table = g.permutation(pages).astype(np.int32)
    native = scatter_pages(pages, pack_pages(k8, ks), table)
    latent = g.integers(0, 256, size=(ctx_tokens, MLA_ROW_BYTES), dtype=np.uint8)
    lens = (first_pos + 1 + np.arange(rows)).astype(np.int32)
    return Workload("config4", seed, dict(q8=q8.reshape(rows, heads, DIM), w=w, native=native, table=table,
                                          lens=lens, latent=latent),
                    dict(rows=rows, heads=heads, ctx=ctx_tokens, topk=TOPK, row_bytes=MLA_ROW_BYTES))


def config5(seed=5, rows=128, heads=64, pool_pages=32768, lo=4096, hi=131072):
    """Decode batch: 128 requests x 1 query (64 heads FP8), context lengths
    round(exp(U(ln 4K, ln 128K))), each request's pages random distinct pages of
    a 2M-token pool; full scoring -> Top-2048 -> slots -> 656-byte row gather."""
    g = rng(seed)
    ctx = np.rint(np.exp(g.uniform(np.log(lo), np.log(hi), size=rows))).astype(np.int32)
    max_pages = int(-(-ctx.max() // PAGE))
    table = np.zeros((rows, max_pages), dtype=np.int32)
    for r in range(rows):
        n = -(-int(ctx[r]) // PAGE)
        table[r, :n] = g.choice(pool_pages, n, replace=False)
    q8, _ = quantize_rows(g.standard_normal((rows * heads, DIM), dtype=np.float32))
    w = g.random((rows, heads), dtype=np.float32)
    k8, ks = quantize_rows(g.standard_normal((pool_pages * PAGE, DIM), dtype=np.float32))
    native = pack_pages(k8, ks)
    latent_rows = pool_pages * PAGE
    return Workload("config5", seed, dict(q8=q8.reshape(rows, heads, DIM), w=w, native=native, table=table,
                                          lens=ctx),
                    dict(rows=rows, heads=heads, topk=TOPK, row_bytes=MLA_ROW_BYTES, latent_rows=latent_rows,
                         max_ctx=int(ctx.max())))


def config5_route(seed=5, rows=128, heads=64, pool_pages=32768, lo=4096, hi=131072, max_context=131072,
                  topk=TOPK, num=1, den=2, sink=64, window=2048):
    """The config5 decode batch (same contexts, native page tables, queries,
    weights and native pool) through the V1 route path of
    sglang/srt/layers/attention/v1_deepseek/runtime.py:417-634 for <= 512 rows:
    center score -> fused route -> fine_table_shared -> stage_tail_shared ->
    fine score -> mask_fine -> topk_transform_512_v2 -> output_ids -> gather,
    with page_fraction num/den (runtime.py:25).

    Each request carries a built index over its complete 1024-token buckets:
    the bucket's tokens in a seeded member order, 16 route pages of 64 members
    per bucket whose FP8 rows are copied into one shared fine pool (the
    reordered table rt maps route page -> fine page through a seeded
    permutation of the pool), and 8 FP8 centers per route page (the float32
    mean of 8 consecutive members, power-of-two scaled).  The route covers
    max_context / 64 pages; the fine pool holds every built page, then 68 tail
    scratch pages per row (Config.width etc.: runtime.py:62-79)."""
    base = config5(seed, rows, heads, pool_pages, lo, hi)
    a = base.arrays
    lens = a["lens"].astype(np.int32)
    assert int(lens.max()) <= max_context and max_context % 4096 == 0
    g = rng(seed + 500)
    P = max_context // PAGE
    take = min(P, max(-(-P * num // den), -(-topk // 64)))
    width = -(-(take * 64 + 64 + 4096) // 256) * 256
    nt = np.zeros((rows, P), np.int32)
    nt[:, :a["table"].shape[1]] = a["table"]
    built = np.maximum(lens.astype(np.int64) - 1, 0) // 1024 * 16
    cap = int(built.sum())
    fine_of = g.permutation(cap).astype(np.int32)
    rt = np.zeros((rows, P), np.int32)
    members = np.full((cap, 64), -1, np.int32)
    fine = np.zeros((cap + rows * 68, PAGE_BYTES), np.uint8)
    centers = np.zeros((max(cap // 8, 1), PAGE_BYTES), np.uint8)
    ctab = np.zeros((rows, P // 8), np.int32)
    nk = a["native"][:, :8192].reshape(pool_pages, PAGE, DIM)
    ns = a["native"][:, 8192:].copy().view(np.float32).reshape(pool_pages, PAGE)
    dec = decode_table()
    fbase = cbase = 0
    for r in range(rows):
        pr = int(built[r])
        if pr == 0:
            continue
        nb = pr // 16
        order = (np.argsort(g.random((nb, 1024)), axis=1) + 1024 * np.arange(nb)[:, None]).reshape(-1)
        ids = fine_of[fbase:fbase + pr]
        rt[r, :pr] = ids
        members[ids] = order.reshape(pr, 64)
        kp, ks = nt[r, order // PAGE], order % PAGE
        k8, sc = nk[kp, ks], ns[kp, ks]
        fine[ids, :8192] = k8.reshape(pr, 8192)
        fine[ids, 8192:] = sc.reshape(pr, PAGE).view(np.uint8)
        mean = (dec[k8] * sc[:, None]).reshape(pr * 8, 8, DIM).sum(axis=1, dtype=np.float32) / np.float32(8.0)
        c8, cs = quantize_rows(mean)
        centers[cbase:cbase + pr // 8] = pack_pages(c8, cs)
        ctab[r, :pr // 8] = cbase + np.arange(pr // 8)
        fbase += pr
        cbase += pr // 8
    out = dict(q8=a["q8"], w=a["w"], native=a["native"], nt=nt, rt=rt, members=members, fine=fine, centers=centers,
               center_table=ctab, lens=lens)
    return Workload("config5_route", seed, out,
                    dict(rows=rows, heads=heads, P=P, CAP=cap, TAKE=take, WIDTH=width, FP=width // 64, topk=topk,
                         num=num, den=den, sink=sink, window=window, row_bytes=MLA_ROW_BYTES,
                         latent_rows=pool_pages * PAGE, max_ctx=int(lens.max())))


def config6(seed=6, pool_pages=32768, buckets=2048):
    """Index build: every complete 1024-token bucket of a 2M-token pool, each
    bucket's 16 pages a distinct slice of a random permutation of the pool's
    pages (every page built once), bucket b starting at logical token b*1024."""
    g = rng(seed)
    if buckets * 16 > pool_pages:
        raise ValueError("buckets need 16 distinct pages each")
    tables = g.permutation(pool_pages)[:buckets * 16].astype(np.int32).reshape(buckets, 16)
    starts = (np.arange(buckets, dtype=np.int64) * 1024).astype(np.int32)
    k8, ks = quantize_rows(g.standard_normal((pool_pages * PAGE, DIM), dtype=np.float32))
    native = pack_pages(k8, ks)
    return Workload("config6", seed, dict(native=native, tables=tables, starts=starts),
                    dict(buckets=buckets, pool_pages=pool_pages))


def config7(seed=7, history=65536, rows=4096, heads=32, sink=64, window=2048, max_take=40):
    """Shared sink + tail chunk (experiments/fine_pool_shared_20261021/
    experiment.py:15-46 shape): one request with `history` published tokens,
    `rows` causal queries (lengths history+1 .. history+rows), `heads` FP8 query
    heads, sink / window, `max_take` history pages per row (64 reordered pages
    whose members are distinct logical positions, the first page the sink),
    indexed_end = history."""
    g = rng(seed)
    pages = -(-(history + rows) // PAGE)
    cap = max(64, max_take)
    k8, ks = quantize_rows(g.standard_normal((pages * PAGE, DIM), dtype=np.float32))
    native = pack_pages(k8, ks)
    nt = g.permutation(pages).astype(np.int32)
    members = np.concatenate([np.arange(64), 64 + g.permutation(history - 64)[:cap * 64 - 64]]).astype(np.int32)
    members = members.reshape(cap, 64)
    nk = native[:, :8192].reshape(-1, PAGE, DIM)
    ns = native[:, 8192:].copy().view(np.float32).reshape(-1, PAGE)
    page, off = nt[members // PAGE], members % PAGE
    reordered = np.zeros((cap, PAGE_BYTES), np.uint8)
    reordered[:, :8192] = nk[page, off].reshape(cap, 8192)
    reordered[:, 8192:] = ns[page, off].view(np.uint8).reshape(cap, 256)
    q8, _ = quantize_rows(g.standard_normal((rows * heads, DIM), dtype=np.float32))
    w = (g.random((rows, heads), dtype=np.float32) / heads).astype(np.float32)
    selected = ((np.arange(max_take)[None] + np.arange(rows)[:, None]) % cap).astype(np.int32)
    return Workload("config7", seed, dict(native=native, nt=nt, members=members, reordered=reordered,
                                          q8=q8.reshape(rows, heads, DIM), w=w, selected=selected,
                                          lens=np.arange(history + 1, history + rows + 1, dtype=np.int32),
                                          takes=np.full(rows, max_take, np.int32)),
                    dict(history=history, rows=rows, heads=heads, sink=sink, window=window, max_take=max_take,
                         cap=cap, pages=pages, indexed_end=history, topk=TOPK))


def decode_table():
    """float32 value of each of the 256 e4m3fn codes (NaN for 0x7f / 0xff)."""
    vals = np.concatenate([_E4M3_POS, [np.nan]]).astype(np.float32)
    return np.concatenate([vals, -vals]).astype(np.float32)
