"""Numpy restatement of the V1 query-indexing path (test infrastructure only).

Integer division follows C / Triton semantics (truncation toward zero) where a
negative operand can occur; see tdiv().
"""
import numpy as np

NEG_INF = np.float32(-np.inf)


def tdiv(a, b):
    """C-style integer division (truncates toward zero)."""
    a = np.asarray(a, dtype=np.int64)
    q = np.abs(a) // b
    return np.where(a < 0, -q, q)


# ----------------------------------------------------------------- FP8
def e4m3_decode(codes):
    """OCP e4m3fn byte -> float32 from the bit fields (1 sign, 4 exponent with
    bias 7, 3 mantissa; exponent 0 is subnormal; 0x7f/0xff are NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return (s * v).astype(np.float32)


# -------------------------------------------------------------- ordering
def score_key(x):
    """Order-preserving uint32 key of fp32 scores; -0.0 folded onto +0.0."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).copy()
    b[b == 0x80000000] = 0
    return np.where(b & 0x80000000, ~b, b | np.uint32(0x80000000)).astype(np.uint32)


def top_order(values, count):
    """Indices of the `count` largest values, value descending, ties by lower index."""
    k = score_key(values)
    return np.argsort(~k, kind="stable")[:count]


def topk_select(row, L, T):
    """Selected raw candidates of one row, ascending, -1 padded to T.
    L <= T takes [0, L) (sglang/kernels/jit/csrc/deepseek_v4/topk_v2.cuh:136-143,
    v1_query.cuh:109-111); otherwise the T largest of row[:L]."""
    out = np.full(T, -1, dtype=np.int64)
    if L <= T:
        out[:L] = np.arange(L)
        return out
    out[:] = np.sort(top_order(row[:L], T))
    return out


# ----------------------------------------------------------------- route
def route(scores, lens, takes, selected, pages, rt, ft, tail_rows, capacity, fill_table):
    """sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:7-49 (in place on
    selected / ft).  Ties between equal page maxima go to the lower page."""
    B = scores.shape[0]
    K = selected.shape[1]
    for b in range(B):
        active = max(int(lens[b]) - 1, 0) // 1024 * 16
        take = int(takes[b])
        if fill_table:
            for j in range(max(take, 0), ft.shape[1]):
                ft[b, j] = capacity + int(tail_rows[b]) * 68 + min(j - take, 67)
        if take >= active:
            selected[b, :] = np.arange(K)
            if fill_table:
                n = max(0, min(take, K))
                ft[b, :n] = rt[b, :n]
            continue
        vals = np.full(pages, NEG_INF, dtype=np.float32)
        if active:
            vals[:active] = np.fmax.reduce(scores[b, : 8 * active].reshape(active, 8), axis=1)
        order = top_order(vals, pages)
        selected[b, :] = order[:K]
        if fill_table:  # every rank < take (v1_query.cuh:44-48), within the table width
            n = max(0, min(take, pages, ft.shape[1]))
            ft[b, :n] = rt[b, order[:n]]


# ------------------------------------------------------------ fused topk
def _bounds(n, window, sink_cap=64):
    sink = min(n, sink_cap)
    tail = max(sink, min(max(n - 1, 0) // 1024 * 1024, max(sink, n - window)))
    return sink, tail


def _map_row(raw, L, row_scores, take, sink, tail, n, members, rt_row, nt_row, sel_row, ft_row):
    """raw -> (logical, physical) of one row (v1_query.cuh:121-139)."""
    raw = np.asarray(raw, dtype=np.int64)
    valid = (raw >= 0) & (raw < L)
    valid &= row_scores[np.where(valid, raw, 0)] != NEG_INF
    lg = np.full(raw.shape, -1, dtype=np.int64)
    fm = valid & (raw < take * 64)
    if fm.any():
        r = raw[fm]
        page = ft_row[r // 64] if ft_row is not None else rt_row[sel_row[r // 64]]
        lg[fm] = members[page, r % 64]
    tm = valid & (raw >= take * 64)
    off = raw[tm] - take * 64
    lg[tm] = np.where(off < sink, off, tail + off - sink)
    ok = valid & (lg >= 0) & (lg < n)
    safe = np.where(ok, lg, 0)
    ph = np.where(ok, nt_row[safe // 64].astype(np.int64) * 64 + safe % 64, -1)
    return np.where(ok, lg, -1).astype(np.int32), ph.astype(np.int32)


def fused_topk(scores, fine_lens, members, rt, nt, selected, lens, takes, T, window, mask, expansion_stride,
               physical_output, bucket_from_rank, fine_table, direct_fine):
    """sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:62-153.  Masks `scores`
    in place; returns dict(physical, logical, raw, expanded)."""
    B, cols = scores.shape
    P = rt.shape[1]
    physical = np.full((B, T), -1, dtype=np.int32)
    logical = np.full((B, T), -1, dtype=np.int32)
    raw_out = np.full((B, T), -1, dtype=np.int32)
    expanded = np.full((B, expansion_stride), -1, dtype=np.int32) if expansion_stride else None
    for b in range(B):
        n, take = int(lens[b]), int(takes[b])
        sink, tail = _bounds(n, window)
        if mask:
            for r in range(take):
                rank = int(selected[b, r])
                if bucket_from_rank:
                    bucket = int(tdiv(rank, 16)) * 1024
                else:
                    page = int(rt[b, rank])
                    bucket = int(tdiv(members[page, 0], 1024)) * 1024
                if bucket < sink or bucket + 1024 > tail:
                    page = int(rt[b, rank])
                    lg = members[page]
                    kill = (lg < sink) | (lg >= tail)
                    cols_r = r * 64 + np.arange(64)
                    ok = cols_r < cols
                    scores[b, cols_r[kill & ok]] = NEG_INF
        L = min(int(fine_lens[b]), cols)
        raw = topk_select(scores[b], L, T)
        lg, ph = _map_row(raw, L, scores[b], take, sink, tail, n, members, rt[b], nt[b], selected[b],
                          fine_table[b] if direct_fine else None)
        logical[b] = lg
        if physical_output:
            physical[b] = ph
            raw_out[b] = raw
        if expansion_stride:
            ex = np.where(lg[:, None] < 0, -1, 4 * lg[:, None].astype(np.int64) + np.arange(4))
            expanded[b, :4 * T] = ex.reshape(-1)
    return dict(physical=physical, logical=logical, raw=raw_out, expanded=expanded)


# ------------------------------------------- the same selections, all rows
# Every-row checks at the benchmark shapes (thousands of rows of 32K+ columns)
# use these batch forms; tests pin them equal to the per-row functions above.
def topk_select_rows(scores, lens, T, chunk=256):
    """topk_select for every row at once: rows with L <= T take [0, L); others
    the T largest of row[:L] by score_key, ties toward the lower index, in
    ascending index order.  Each column gets the unique 64-bit composite
    (key << 32) | (2^32 - 1 - index) (padding past L is 0, below every real
    composite), and a row's T winners are the composites at or above its
    T-th largest one (np.partition)."""
    scores = np.asarray(scores, dtype=np.float32)
    B, cols = scores.shape
    lens = np.minimum(np.asarray(lens, dtype=np.int64), cols)
    out = np.full((B, T), -1, dtype=np.int64)
    col = np.arange(cols, dtype=np.uint64)
    for b0 in range(0, B, chunk):
        L = lens[b0:b0 + chunk]
        big = np.nonzero(L > T)[0]
        for k in np.nonzero(L <= T)[0]:
            out[b0 + k, :max(int(L[k]), 0)] = np.arange(max(int(L[k]), 0))
        if big.size == 0:
            continue
        comp = (score_key(scores[b0 + big]).astype(np.uint64) << np.uint64(32)) | (np.uint64(0xffffffff) - col)
        comp[col[None, :] >= L[big, None].astype(np.uint64)] = 0
        thr = np.partition(comp, cols - T, axis=1)[:, cols - T]
        _, j = np.nonzero(comp >= thr[:, None])
        out[b0 + big] = j.reshape(big.size, T)
    return out


def transform_topk_rows(scores, seq_lens, page_table, T, page_bits):
    """transform_topk with the batch selection: returns (page_indices, raw)."""
    raws = topk_select_rows(scores, np.minimum(np.asarray(seq_lens, np.int64), scores.shape[1]), T)
    ok = raws >= 0
    safe = np.where(ok, raws, 0)
    entry = np.take_along_axis(np.asarray(page_table, np.int64), safe >> page_bits, axis=1)
    out = np.where(ok, (entry << page_bits) | (safe & ((1 << page_bits) - 1)), -1)
    return out.astype(np.int32), raws.astype(np.int32)


def v1_mask_rows(scores, members, rt, selected, lens, takes, window, bucket_from_rank, chunk=128):
    """fused_topk's in-place sink/tail mask (v1_query.cuh:71-107) for every
    row at once: rank r < take of a row whose bucket overlaps the sink or the
    tail gets -inf at the columns r * 64 + j whose member lies outside
    [sink, tail)."""
    B, cols = scores.shape
    K = selected.shape[1]
    r = np.arange(K)
    colr = r[:, None] * 64 + np.arange(64)[None, :]
    for b0 in range(0, B, chunk):
        b1 = min(B, b0 + chunk)
        n = np.asarray(lens[b0:b1], np.int64)
        sink = np.minimum(n, 64)
        tail = np.maximum(sink, np.minimum(np.maximum(n - 1, 0) // 1024 * 1024, np.maximum(sink, n - window)))
        live = r[None, :] < np.asarray(takes[b0:b1], np.int64)[:, None]
        rank = np.where(live, np.asarray(selected[b0:b1], np.int64), 0)
        page = np.take_along_axis(np.asarray(rt[b0:b1], np.int64), rank, axis=1)
        if bucket_from_rank:
            bucket = tdiv(rank, 16) * 1024
        else:
            bucket = tdiv(members[page, 0], 1024) * 1024
        cond = live & ((bucket < sink[:, None]) | (bucket + 1024 > tail[:, None]))
        lg = members[page]
        kill = cond[:, :, None] & ((lg < sink[:, None, None]) | (lg >= tail[:, None, None])) & (colr < cols)[None]
        bi, ri, ji = np.nonzero(kill)
        scores[b0 + bi, ri * 64 + ji] = NEG_INF


def fused_topk_rows(scores, fine_lens, members, rt, nt, selected, lens, takes, T, window, mask, expansion_stride,
                    physical_output, bucket_from_rank, fine_table, direct_fine):
    """fused_topk with the batch mask and selection (same outputs, same
    in-place mask)."""
    B, cols = scores.shape
    if mask:
        v1_mask_rows(scores, members, rt, selected, lens, takes, window, bucket_from_rank)
    L = np.minimum(np.asarray(fine_lens, np.int64), cols)
    raws = topk_select_rows(scores, L, T)
    physical = np.full((B, T), -1, dtype=np.int32)
    logical = np.full((B, T), -1, dtype=np.int32)
    raw_out = np.full((B, T), -1, dtype=np.int32)
    expanded = np.full((B, expansion_stride), -1, dtype=np.int32) if expansion_stride else None
    for b in range(B):
        n, take = int(lens[b]), int(takes[b])
        sink, tail = _bounds(n, window)
        lg, ph = _map_row(raws[b], int(L[b]), scores[b], take, sink, tail, n, members, rt[b], nt[b], selected[b],
                          fine_table[b] if direct_fine else None)
        logical[b] = lg
        if physical_output:
            physical[b] = ph
            raw_out[b] = raws[b]
        if expansion_stride:
            ex = np.where(lg[:, None] < 0, -1, 4 * lg[:, None].astype(np.int64) + np.arange(4))
            expanded[b, :4 * T] = ex.reshape(-1)
    return dict(physical=physical, logical=logical, raw=raw_out, expanded=expanded)


def transform_topk(scores, seq_lens, page_table, T, page_bits):
    """topk_impl.cuh:156-190 transform after selection: returns (page_indices, raw)."""
    B, cols = scores.shape
    out = np.full((B, T), -1, dtype=np.int64)
    raws = np.full((B, T), -1, dtype=np.int64)
    mask = (1 << page_bits) - 1
    for b in range(B):
        L = min(int(seq_lens[b]), cols)
        raw = topk_select(scores[b], L, T)
        raws[b] = raw
        ok = raw >= 0
        r = raw[ok]
        out[b, ok] = (page_table[b, r >> page_bits].astype(np.int64) << page_bits) | (r & mask)
    return out.astype(np.int32), raws.astype(np.int32)


# ------------------------------------------------------ unfused mask / map
def expand_logical(logical, out, block=None):
    """kernels.py:594-600 (the unfused C4 x4 expansion, runtime.py:638-641), in
    place on out [rows, stride]: columns j < min(stride, block) become
    4 * logical[r, j // 4] + j % 4 when j < 4 * topk and that index is >= 0,
    else -1 (int32, wrapping); columns past block are left as they are."""
    logical = np.asarray(logical, np.int32)
    rows, topk = logical.shape
    stride = out.shape[1]
    cols = stride if block is None else min(stride, block)
    j = np.arange(cols)
    src = np.full((rows, cols), -1, np.int64)
    inside = j < 4 * topk
    src[:, inside] = logical[:, j[inside] // 4]
    val = ((src.astype(np.uint32) * np.uint32(4)) + (j % 4).astype(np.uint32)).view(np.int32)
    out[:, :cols] = np.where(src >= 0, val, -1)
    return out


def mask_fine(scores, selected, rt, members, lens, takes, width, sink_cap, window):
    """sglang/srt/layers/attention/v1_deepseek/kernels.py:444-472 (in place)."""
    B = scores.shape[0]
    j = np.arange(width)
    for b in range(B):
        n, take = int(lens[b]), int(takes[b])
        sink, tail = _bounds(n, window, sink_cap)
        count = take * 64 + sink + n - tail
        fine = j < take * 64
        lg = np.full(width, -1, dtype=np.int64)
        if fine.any():
            jj = j[fine]
            pages = rt[b, selected[b, jj // 64]]
            lg[fine] = members[pages, jj % 64]
        good = (j < count) & (~fine | ((lg >= sink) & (lg < tail)))
        scores[b, :width][~good] = NEG_INF


def output_ids(raw, scores, members, rt, nt, selected, lens, takes, width, topk, sink_cap, window, map_physical,
               direct_fine, ft):
    """sglang/srt/layers/attention/v1_deepseek/kernels.py:323-376."""
    B = raw.shape[0]
    out = np.full((B, topk), -1, dtype=np.int32)
    logical = np.full((B, topk), -1, dtype=np.int32)
    for b in range(B):
        n, take = int(lens[b]), int(takes[b])
        sink, tail = _bounds(n, window, sink_cap)
        for j in range(topk):
            rw = int(raw[b, j])
            if not (0 <= rw < width):
                continue
            if rw < take * 64:
                page = int(ft[b, rw // 64]) if direct_fine else int(rt[b, int(selected[b, rw // 64])])
                lg = int(members[page, rw % 64])
            else:
                off = rw - take * 64
                lg = off if off < sink else tail + off - sink
            if scores[b, rw] == NEG_INF or not (0 <= lg < n):
                continue
            logical[b, j] = lg
            if map_physical:
                out[b, j] = int(nt[b, lg // 64]) * 64 + lg % 64
    return out, logical


# -------------------------------------------------------------- metadata
def geometry(n, topk, num, den, sink_cap, window):
    """kernels.py:224-245, 568-582: (pages, take, sink, tail, fine)."""
    pages = max(n - 1, 0) // 1024 * 16
    take = min(pages, max((pages * num + den - 1) // den, -(-topk // 64)))
    sink, tail = _bounds(n, window, sink_cap)
    return pages, take, sink, tail, take * 64 + sink + n - tail


def query_metadata(lens, nt, topk, num, den, sink_cap, window):
    """kernels.py:568-591: (fine_lens, takes, dg_lens, center_lens, tail_rows)."""
    B, NP = nt.shape
    outs = [np.zeros(B, np.int32) for _ in range(5)]
    for r in range(B):
        n = int(lens[r])
        pages, take, sink, tail, fine = geometry(n, topk, num, den, sink_cap, window)
        outs[0][r], outs[1][r], outs[2][r], outs[3][r] = fine, take, max(fine, 1), max(pages * 8, 1)
        same = True
        for i in range(128):
            page = 0 if i == 0 else tail // 64 + i - 1
            valid = n > 0 and (i == 0 or page < (n + 63) // 64) and page < NP
            mine = int(nt[r, page]) if valid else -1
            first = int(nt[0, page]) if valid else -1
            same &= mine == first
        outs[4][r] = 0 if (n == int(lens[0]) and same) else r
    return tuple(outs)


def fine_table(rt, selected, takes, fp, capacity, scratch, tail_rows=None):
    """kernels.py:379-404 (tail_rows None) and :488-514."""
    B = rt.shape[0]
    ft = np.zeros((B, fp), dtype=np.int32)
    for b in range(B):
        take = int(takes[b])
        owner = b if tail_rows is None else int(tail_rows[b])
        for j in range(fp):
            if j < take:
                ft[b, j] = rt[b, int(selected[b, j])]
            else:
                ft[b, j] = capacity + owner * scratch + min(max(j - take, 0), scratch - 1)
    return ft


def stage_tail(native, nt, lens, fine, capacity, scratch, sink_cap, window, tail_rows=None, rows=None,
               indexed_end=None):
    """kernels.py:518-564 (tail_rows None: :407-441) on byte pools [pages, 8448]
    (in place on fine).  With indexed_end the tail starts at the published index
    end (experiments/tail_union_lab_20261021/baseline_published.py:38-41)."""
    B = nt.shape[0] if rows is None else rows
    nat_k = native[:, :8192].reshape(-1, 64, 128)
    nat_s = native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    for row in range(B):
        if tail_rows is not None and int(tail_rows[row]) != row:
            continue
        n = int(lens[row])
        if indexed_end is None:
            sink, tail = _bounds(n, window, sink_cap)
        else:
            sink, tail, _ = union_bounds(n, int(indexed_end), sink_cap, window)
        count = sink + n - tail
        for p in range(scratch):
            if not (p * 64 < count or p == 0):
                continue
            dst = capacity + row * scratch + p
            kb = np.zeros((64, 128), dtype=np.uint8)
            sb = np.zeros(64, dtype=np.float32)
            for o in range(64):
                i = p * 64 + o
                if i < count:
                    lg = i if i < sink else tail + i - sink
                    page = int(nt[row, lg // 64])
                    kb[o] = nat_k[page, lg % 64]
                    sb[o] = nat_s[page, lg % 64]
            fine[dst, :8192] = kb.reshape(-1)
            fine[dst, 8192:] = sb.view(np.uint8)


def stage_tail_rows(native, nt, lens, fine, capacity, scratch, sink_cap, window, row_bytes, tail_rows=None):
    """stage_tail(_shared) (kernels.py:518-564, :407-441) over pages of 64 rows
    of row_bytes each, one row per token (in place on fine)."""
    nat = native.reshape(native.shape[0], 64, row_bytes)
    out = fine.reshape(fine.shape[0], 64, row_bytes)
    for row in range(nt.shape[0]):
        if tail_rows is not None and int(tail_rows[row]) != row:
            continue
        n = int(lens[row])
        sink, tail = _bounds(n, window, sink_cap)
        count = sink + n - tail
        for p in range(scratch):
            if not (p * 64 < count or p == 0):
                continue
            dst = capacity + row * scratch + p
            out[dst] = 0
            for o in range(min(64, max(count - p * 64, 0))):
                i = p * 64 + o
                lg = i if i < sink else tail + i - sink
                out[dst, o] = nat[int(nt[row, lg // 64]), lg % 64]


# ------------------------------------------------------------------ sort
def sort_f32(perm, keys, n, groups, heads=1, head_stride=4096):
    """sglang/srt/layers/attention/v1_native/fused_grouping.py:64-76: returns O."""
    out = np.array(perm, copy=True)
    for h in range(heads):
        for g in range(groups):
            base = h * head_stride + g * n
            order = top_order(keys[base:base + n], n)
            out[base:base + n] = perm[base + order]
    return out


def sort_i64(perm, keys, n):
    """Same rule for signed int64 keys: descending, ties by ascending position."""
    out = np.array(perm, copy=True)
    for g in range(len(keys) // n):
        k = keys[g * n:(g + 1) * n].astype(np.int64)
        order = np.lexsort((np.arange(n), ~k))
        out[g * n:(g + 1) * n] = perm[g * n + order]
    return out


# ---------------------------------------------------------- page manager
def fingerprint(tmp, mapping):
    """kernels.py:57-69: int64 [pages, 2] of byte and member weighted sums."""
    pages, nbytes = tmp.shape
    i = np.arange(nbytes, dtype=np.int64)
    m_i = np.arange(64, dtype=np.int64)
    out = np.zeros((pages, 2), dtype=np.int64)
    for p in range(pages):
        x = tmp[p].astype(np.int64)
        m = mapping[p].astype(np.int64)
        out[p, 0] = int((x * (i + 1)).sum()) + int(m.sum()) * 104729
        out[p, 1] = int((x * ((i + 7) * 1000003)).sum()) + int((m * (m_i + 1) * 65537).sum())
    return out


def match_pages(tmp, mapping, hashes_tmp, fine, members, hashes, refs, capacity):
    """kernels.py:72-113: lowest live page with equal fingerprints and equal
    bytes + members, else -1."""
    out = np.full(tmp.shape[0], -1, dtype=np.int32)
    live = np.nonzero(refs[:capacity] > 0)[0]
    for p in range(tmp.shape[0]):
        for j in live:
            if hashes[j, 0] == hashes_tmp[p, 0] and hashes[j, 1] == hashes_tmp[p, 1]:
                if np.array_equal(fine[j], tmp[p]) and np.array_equal(members[j], mapping[p]):
                    out[p] = j
                    break
    return out


def allocate(lease, match, free, count, refs, tables):
    """kernels.py:116-131 (in place on free-stack count / refs / tables).
    Returns (new_count, fresh) or raises on exhaustion (the reference asserts)."""
    fresh = match < 0
    rank = np.cumsum(fresh) - 1
    needed = int(fresh.sum())
    if count < needed:
        raise RuntimeError("V1 DeepSeek page arena exhausted")
    pages = len(match)
    dst = np.where(fresh, free[np.clip(count - 1 - rank, 0, None)], match)
    np.add.at(refs, dst, 1)
    tables[lease * pages:(lease + 1) * pages] = dst
    return count - needed, fresh


def publish(lease, tmp, centers_tmp, mapping, hash_tmp, tables, fresh, fine, centers, members, hashes):
    """kernels.py:134-167 (in place).  Centers: 8 per page, 128 FP8 bytes plus
    one fp32 scale each, to center index lease*pages*8 + p*8 + g."""
    pages = len(fresh)
    for p in range(pages):
        if fresh[p]:
            dst = int(tables[lease * pages + p])
            fine[dst] = tmp[p]
            members[dst] = mapping[p]
            hashes[dst] = hash_tmp[p]
        for g in range(8):
            sc = p * 8 + g
            dc = lease * pages * 8 + sc
            centers[dc // 64, (dc % 64) * 128:(dc % 64) * 128 + 128] = \
                centers_tmp[sc // 64, (sc % 64) * 128:(sc % 64) * 128 + 128]
            centers[dc // 64, 8192 + 4 * (dc % 64):8192 + 4 * (dc % 64) + 4] = \
                centers_tmp[sc // 64, 8192 + 4 * (sc % 64):8192 + 4 * (sc % 64) + 4]


def release(table, refs, free, count):
    """kernels.py:170-179, decrements in table order; returns the new count."""
    dead = []
    for page in table:
        old = int(refs[page])
        refs[page] = old - 1
        if old == 1:
            dead.append(int(page))
    free[count:count + len(dead)] = dead
    return count + len(dead)


def live_index(pool_keys, refs):
    """key -> live pages (refs > 0) in page order."""
    live = {}
    for p in np.nonzero(refs > 0)[0]:
        live.setdefault(int(pool_keys[p]), []).append(int(p))
    return live


def insert_request_inplace(pool, pool_keys, refs, free, count, live, keys, tmp, s, e, table):
    """One request (entries s..e): match_pages (kernels.py:72-113: lowest live
    page with equal key and bytes), allocate (:116-131: free[count-1-rank],
    refs += 1), publish (:134-167: bytes and key to fresh pages), in place.
    Returns the new count; raises RuntimeError before any change when the
    free stack is too short."""
    match = np.full(e - s, -1, dtype=np.int64)
    for i in range(s, e):
        for p in live.get(int(keys[i]), ()):
            if np.array_equal(pool[p], tmp[i]):
                match[i - s] = p
                break
    fresh = match < 0
    need = int(fresh.sum())
    if count < need:
        raise RuntimeError("V1 DeepSeek page arena exhausted")
    rank = np.cumsum(fresh) - 1
    dst = np.where(fresh, free[np.clip(count - 1 - rank, 0, None)], match)
    np.add.at(refs, dst, 1)
    table[s:e] = dst
    for i in np.flatnonzero(fresh) + s:
        p = int(table[i])
        pool[p] = tmp[i]
        pool_keys[p] = keys[i]
        pages = live.setdefault(int(keys[i]), [])
        pages.insert(int(np.searchsorted(pages, p)), p)
    return count - need


def page_insert_batch(pool, pool_keys, refs, free, count, keys, tmp, req):
    """match_pages -> allocate -> publish (kernels.py:72-167) called request
    after request (runtime.py:230-270) with an int64 key in place of the
    (h0, h1) fingerprint.  An entry takes the lowest live page (refs > 0) with
    equal key and bytes; entries of one request are not matched against each
    other; unmatched entries take free[count-1-rank].  All or nothing: raises
    RuntimeError (state untouched) when the free stack runs out.  Returns
    (table, pool, pool_keys, refs, free, new_count) as new arrays."""
    pool, pool_keys, refs, free = pool.copy(), pool_keys.copy(), refs.copy(), free.copy()
    n = len(keys)
    table = np.empty(n, dtype=np.int32)
    live = live_index(pool_keys, refs)
    bounds = np.flatnonzero(np.diff(np.asarray(req, dtype=np.int64))) + 1
    starts = np.concatenate([[0], bounds]).astype(np.int64) if n else np.zeros(0, np.int64)
    ends = np.concatenate([bounds, [n]]).astype(np.int64) if n else np.zeros(0, np.int64)
    for s, e in zip(starts, ends):
        count = insert_request_inplace(pool, pool_keys, refs, free, count, live, keys, tmp, s, e, table)
    return table, pool, pool_keys, refs, free, count


def page_release_batch(pages, refs, free, count):
    """release (kernels.py:170-179) of a list of pages in list order; raises
    RuntimeError (state untouched) when a page has no reference left or is out
    of range.  Returns (refs, free, new_count) as new arrays."""
    refs, free = refs.copy(), free.copy()
    pages = np.asarray(pages, dtype=np.int64)
    if len(pages):
        if pages.min() < 0 or pages.max() >= len(refs):
            raise RuntimeError("page release of an id out of range")
        u, c = np.unique(pages, return_counts=True)
        if np.any(refs[u] < c):
            raise RuntimeError("page release underflow")
    count = release(pages, refs, free, count)
    return refs, free, count


# ---------------------------------------------------------------- gather
def gather_slots(k_pool, v_pool, req, ids, head):
    """sglang/srt/layers/attention/v1_native/kernels.py:62-77 -> (kg, vg) [rows, top, 1, 128]."""
    valid = ids >= 0
    slots = req[np.where(valid, ids, 0)]
    kg = np.where(valid[..., None], k_pool[slots, head], 0).astype(k_pool.dtype)
    vg = np.where(valid[..., None], v_pool[slots, head], 0).astype(v_pool.dtype)
    return kg[:, :, None, :], vg[:, :, None, :]


def physical_rows(ids, table=None, page_bits=0):
    """ids -> physical rows (-1 stays -1); table None / shared 1-D / per-row."""
    ids = np.asarray(ids, dtype=np.int64)
    if table is None:
        return ids
    valid = ids >= 0
    e = np.where(valid, ids >> page_bits, 0)
    t = table[e] if table.ndim == 1 else np.take_along_axis(table, e, axis=1)
    phys = (t.astype(np.int64) << page_bits) | (ids & ((1 << page_bits) - 1))
    return np.where(valid, phys, -1)


def gather_rows(pool, ids, table=None, page_bits=0):
    """Rows of `pool` at the physical ids; -1 and ids outside the pool give
    zero rows (this build's contract for ids the reference leaves undefined)."""
    phys = physical_rows(ids, table, page_bits)
    ok = (phys >= 0) & (phys < len(pool))
    out = pool[np.where(ok, phys, 0)]
    out[~ok] = 0
    return out


# ---------------------------------------------------------------- score
def paged_logits(q8, w, native, block_table, lens, max_len, relu=True, clean=True, magnitude=False):
    """Dequantised reference of the FP8 paged index logits (fp64 accumulation):
    logit[r,j] = sum_h w[r,h] * relu(q[r,h] . k[j]) * s_k[j] for j < lens[r]
    (sglang/srt/layers/attention/v1_deepseek/kernels.py:310-313; weighted
    head sum, then the key scale).  Columns >= lens[r] are -inf (clean).
    magnitude=True returns sum_h |w| sum_d |q k| s_k instead: the scale of the
    terms, which bounds the rounding of any fp32 accumulation order."""
    rows, H, D = q8.shape
    qf = e4m3_decode(q8).astype(np.float64)
    kk = native[:, :8192].reshape(-1, 64, 128)
    ks = native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    out = np.full((rows, max_len), -np.inf if clean else 0.0, dtype=np.float64)
    for r in range(rows):
        n = min(int(lens[r]), max_len)
        if n <= 0:
            continue
        tab = block_table[r] if block_table.ndim == 2 else block_table
        j = np.arange(n)
        pages = tab[j // 64]
        k = e4m3_decode(kk[pages, j % 64]).astype(np.float64)
        s = ks[pages, j % 64].astype(np.float64)
        if magnitude:
            out[r, :n] = (np.abs(w[r].astype(np.float64))[:, None] * (np.abs(qf[r]) @ np.abs(k).T)).sum(axis=0) * s
            continue
        dots = qf[r] @ k.T  # [H, n]
        if relu:
            dots = np.maximum(dots, 0.0)
        out[r, :n] = (w[r].astype(np.float64)[:, None] * dots).sum(axis=0) * s
    return out


# --------------------------------------------- scoring without DeepGEMM
# The reference's Triton fallbacks when DeepGEMM is absent or the query
# optimisations are off (runtime.py:450-466, 565-590).
def reduce_centers(logits, lens, maxp):
    """sglang/srt/layers/attention/v1_deepseek/kernels.py:475-486: page p of a
    row scores the max of its 8 center logits (columns 8p..8p+7) for p below
    pages(n) = max(n-1, 0) // 1024 * 16, else -inf; [rows, maxp] fp32."""
    rows = logits.shape[0]
    out = np.full((rows, maxp), NEG_INF, dtype=np.float32)
    for r in range(rows):
        pages = min(tdiv(max(int(lens[r]) - 1, 0), 1024) * 16, maxp)
        if pages > 0:
            out[r, :pages] = np.fmax.reduce(np.asarray(logits[r, :pages * 8], dtype=np.float32).reshape(pages, 8),
                                            axis=1)
    return out


def coarse(q8, w, centers, table, lens, maxp, relu=True):
    """kernels.py:182-221: center page table[r, b] holds the 64 centers of
    pages 8b..8b+7 (8 each); a page scores the max of its centers'
    sum_h w relu(q . c) s_c, for pages below pages(n), else -inf.  Restated
    as the center logits of each row's pages(n) * 8 centers followed by
    reduce_centers."""
    pages = np.array([min(tdiv(max(int(n) - 1, 0), 1024) * 16, maxp) for n in lens], dtype=np.int64)
    logits = paged_logits(q8, w, centers, np.asarray(table), pages * 8, maxp * 8, relu=relu)
    return reduce_centers(logits, lens, maxp)


def fine(q8, w, fine_pool, native, members, rt, nt, selected, lens, takes, width, sink_cap, window, relu=True,
         magnitude=False):
    """kernels.py:248-320: candidate i of a row is slot i % 64 of fine page
    rt[selected[i // 64]] for i < take * 64 (kept when its logical position
    members[page, slot] lies in [sink, tail) and below n), then the sink and
    tail tokens read straight from the native pool (logical i' for
    i' = i - take * 64 < sink, else tail + i' - sink, kept below count);
    score = sum_h w relu(q . k) s_k in fp64, -inf where not kept.
    magnitude=True gives sum_h |w| sum_d |q k| s_k at the kept candidates."""
    rows = q8.shape[0]
    qf = e4m3_decode(q8).astype(np.float64)
    pools = (fine_pool, native)
    keys = [p[:, :8192].reshape(-1, 64, 128) for p in pools]
    scales = [p[:, 8192:].copy().view(np.float32).reshape(-1, 64) for p in pools]
    out = np.full((rows, width), -np.inf, dtype=np.float64)
    for r in range(rows):
        n, take = int(lens[r]), int(takes[r])
        sink, tail = _bounds(n, window, sink_cap)
        count = take * 64 + sink + n - tail
        for i in range(min(width, max(count, 0))):
            if i < take * 64:
                src, page, slot = 0, int(rt[r, int(selected[r, i // 64])]), i % 64
                logical = int(members[page, slot])
                keep = sink <= logical < tail and logical < n
            else:
                off = i - take * 64
                logical = off if off < sink else tail + off - sink
                src, page, slot = 1, int(nt[r, logical // 64]), logical % 64
                keep = logical < n
            if not keep:
                continue
            k = e4m3_decode(keys[src][page, slot]).astype(np.float64)
            s = float(scales[src][page, slot])
            if magnitude:
                out[r, i] = float((np.abs(w[r].astype(np.float64)) * (np.abs(qf[r]) @ np.abs(k))).sum()) * s
                continue
            dots = qf[r] @ k
            if relu:
                dots = np.maximum(dots, 0.0)
            out[r, i] = float((w[r].astype(np.float64) * dots).sum()) * s
    return out


# ------------------------------------------------------------ index build
# The producer of the pages the query path reads: per 1024-token bucket
# (16 native pages), unit vectors, a balanced cosine bisection into groups of
# 8 (runtime.py:171-216), then the permuted pages, member map and FP8 group
# centers (kernels.py:33-54).  The reference's 128-wide fp32 sums are Triton
# reductions whose order is not specified; this build fixes its own order
# (reduce128 below) and the GPU kernels reproduce it bit for bit.
BUILD_TOKENS = 1024
BUILD_LEVELS = (1024, 512, 256, 128, 64, 32, 16)


def reduce128(prod):
    """Sum over the last axis (a multiple of 4 wide) in this build's order:
    four partial sums over dims d = r (mod 4), each taken in ascending d with
    one fp32 rounding per addition, then (p0 + p1) + (p2 + p3)."""
    prod = np.asarray(prod, dtype=np.float32)
    acc = np.zeros(prod.shape[:-1] + (4,), dtype=np.float32)
    for d in range(0, prod.shape[-1], 4):
        acc = (acc + prod[..., d:d + 4]).astype(np.float32)
    return ((acc[..., 0] + acc[..., 1]) + (acc[..., 2] + acc[..., 3])).astype(np.float32)


def bucket_tokens(native, table):
    """FP8 key bytes [1024, 128] and fp32 scales [1024] of a bucket's tokens:
    token i lives in native page table[i // 64], slot i % 64."""
    pages = np.asarray(table, dtype=np.int64)[np.arange(BUILD_TOKENS) // 64]
    slot = np.arange(BUILD_TOKENS) % 64
    codes = native[pages[:, None], slot[:, None] * 128 + np.arange(128)[None, :]]
    scales = native[:, 8192:].copy().view(np.float32)[pages, slot]
    return codes, scales


def unit_vectors(codes, scales):
    """kernels.py:17-28: x_d = fl(c_d * s), unit_d = fl(x_d / max(||x||, 1e-12)),
    the reference's order of operations; ||x|| = sqrt(reduce128(x * x)) (the
    one order the reference leaves open: tl.sum's)."""
    c = e4m3_decode(codes)
    s = np.asarray(scales, dtype=np.float32)
    x = (c * s[:, None]).astype(np.float32)
    norm = np.sqrt(reduce128((x * x).astype(np.float32))).astype(np.float32)
    m = np.maximum(norm, np.float32(1e-12))
    return (x / m[:, None]).astype(np.float32)


def build_initialize(native, table):
    """kernels.py:9-30 for one active bucket: unit [1024, 128], perm = 0..1023."""
    codes, scales = bucket_tokens(native, table)
    return unit_vectors(codes, scales), np.arange(BUILD_TOKENS, dtype=np.int32)


def group_dots(unit, perm, anchor, scores, n, start, mode):
    """fused_grouping.py:38-52 (one head, len(perm) positions), in place on scores:
    mode 0 dots each member with its group's first member, modes 1 / 2 with
    anchor[group, mode - 1]; mode 2 subtracts the previous scores."""
    i = np.arange(len(perm))
    group = i // n
    ids = np.asarray(perm, dtype=np.int64)[i] - start
    if mode == 0:
        anc = np.asarray(perm, dtype=np.int64)[group * n] - start
    else:
        anc = np.asarray(anchor, dtype=np.int64)[group, mode - 1] - start
    value = reduce128((unit[ids] * unit[anc]).astype(np.float32))
    if mode == 2:
        value = (value - np.asarray(scores, dtype=np.float32)).astype(np.float32)
    scores[:] = value


def group_anchor(perm, anchor, scores, n, slot):
    """fused_grouping.py:54-61: anchor[g, slot] = member at the group's first
    minimum score (-0.0 == +0.0)."""
    for g in range(len(perm) // n):
        sc = np.asarray(scores[g * n:(g + 1) * n], dtype=np.float32)
        anchor[g, slot] = perm[g * n + int(np.argmin(sc))]


def group_bisect(unit, start=0):
    """runtime.py:183-215: for n = 1024 .. 16, three dots / two anchors per
    group of n, then a stable descending sort of each group by the last
    scores (so the next level's groups are its halves).  Returns the final
    member order (start + token index) and the anchors [levels, groups, 2]."""
    perm = (start + np.arange(BUILD_TOKENS)).astype(np.int32)
    scores = np.zeros(BUILD_TOKENS, dtype=np.float32)
    anchors = np.full((len(BUILD_LEVELS), 64, 2), -1, dtype=np.int32)
    for li, n in enumerate(BUILD_LEVELS):
        anchor = np.zeros((BUILD_TOKENS // n, 2), dtype=np.int32)
        for mode in (0, 1, 2):
            group_dots(unit, perm, anchor, scores, n, start, mode)
            if mode < 2:
                group_anchor(perm, anchor, scores, n, mode)
        anchors[li, :BUILD_TOKENS // n] = anchor
        perm = sort_f32(perm, scores, n, BUILD_TOKENS // n)
    return perm, anchors


_E4M3_POS = np.where(np.arange(127) >> 3 == 0, (np.arange(127) & 7) / 8.0 * 2.0 ** -6,
                     (1 + (np.arange(127) & 7) / 8.0) * 2.0 ** ((np.arange(127) >> 3) - 7.0))


def e4m3_encode(x):
    """Round-to-nearest-even float32 -> e4m3fn byte (|x| <= 448)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    assert a.size == 0 or float(a.max()) <= 448.0
    hi = np.clip(np.searchsorted(_E4M3_POS, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dl, dh = a - _E4M3_POS[lo], _E4M3_POS[hi] - a
    pick_hi = (dh < dl) | ((dh == dl) & ((hi & 1) == 0))
    return np.where(pick_hi, hi, lo).astype(np.uint8) | (np.signbit(x).astype(np.uint8) << 7)


def center_scale(amax):
    """Smallest power of two >= fl(max(amax, 1e-4) / 448) (the exp2(ceil(log2(.)))
    of kernels.py:46-48, exactly)."""
    v = (np.maximum(np.asarray(amax, dtype=np.float32), np.float32(1e-4)) / np.float32(448.0)).astype(np.float32)
    m, e = np.frexp(v)
    e = np.where(m == 0.5, e - 1, e)
    return np.ldexp(np.float32(1.0), e).astype(np.float32)


def build_assemble(native, table, ids, start):
    """kernels.py:33-54 for one active bucket: TMP [16, 8448] (page p slot i =
    token ids[p*64 + i] with its scale), MAP [16, 64] = start + id, and 128
    FP8 centers (mean of 8 consecutive members, power-of-two scale) packed as
    CENTERS [2, 8448].  The mean is the sum over the 8 members in order, one
    fp32 rounding per product and per addition, times 1/8."""
    codes, scales = bucket_tokens(native, table)
    ids = np.asarray(ids, dtype=np.int64)
    tmp = np.zeros((16, 8448), dtype=np.uint8)
    tmp[:, :8192] = codes[ids].reshape(16, 8192)
    tmp[:, 8192:] = scales[ids].astype(np.float32).reshape(16, 64).view(np.uint8)
    mapping = (start + ids).astype(np.int32).reshape(16, 64)
    x = (e4m3_decode(codes[ids]) * scales[ids][:, None]).astype(np.float32).reshape(128, 8, 128)
    acc = x[:, 0]
    for j in range(1, 8):
        acc = (acc + x[:, j]).astype(np.float32)
    mean = (acc * np.float32(0.125)).astype(np.float32)
    cs = center_scale(np.abs(mean).max(axis=1))
    centers = np.zeros((2, 8448), dtype=np.uint8)
    centers[:, :8192] = e4m3_encode((mean / cs[:, None]).astype(np.float32)).reshape(2, 8192)
    centers[:, 8192:] = cs.reshape(2, 64).view(np.uint8)
    return tmp, mapping, centers


def index_build(native, table, start):
    """One bucket's producer chain (runtime.py:171-228 up to assemble):
    returns (perm, tmp, mapping, centers)."""
    unit, _ = build_initialize(native, table)
    perm, _ = group_bisect(unit, 0)
    tmp, mapping, centers = build_assemble(native, table, perm, start)
    return perm, tmp, mapping, centers


# ------------------------------------------------- shared sink + tail union
def union_bounds(n, end, S, W):
    """experiments/tail_union_lab_20261021/union.py:10-14: (s, t, count)."""
    s = min(n, S)
    t = max(s, min(min(max(end, 0), n), max(s, n - W)))
    return s, t, s + n - t


def union_pages(lens, end, S, W):
    """union.py:18-24: (sp, tp, ep, total) of the union of every row's pages."""
    first, last = int(lens[0]), int(lens[-1])
    sp = (min(last, S) + 63) // 64
    tp = max(sp, union_bounds(first, end, S, W)[1] // 64)
    ep = (last + 63) // 64
    return sp, tp, ep, sp + max(ep - tp, 0)


def stage_union(src, nt, lens, end, dst, S, W):
    """union.py:16-40 on byte pools [pages, 8448]: union page b <- source page
    nt[b if b < sp else tp + b - sp] for b < min(total, capacity), in place on
    dst; returns (meta [rows, 3], desc [4])."""
    sp, tp, ep, total = union_pages(lens, end, S, W)
    for b in range(min(total, dst.shape[0])):
        lp = b if b < sp else tp + b - sp
        dst[b] = src[int(nt[lp])]
    meta = np.array([union_bounds(int(n), end, S, W) for n in lens], np.int32).reshape(-1, 3)
    return meta, np.array([sp, tp, ep, total], np.int32)


def union_reconstruct(union, meta, desc, scratch):
    """union.py:26-42 (reconstruct_for_test): each row's candidates read from the
    union into its own scratch pages (row * scratch + p), the layout the per-row
    staging writes; pages past the count are not written (None)."""
    rows = meta.shape[0]
    uk = union[:, :8192].reshape(-1, 64, 128)
    us = union[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    out = {}
    sp, tp = int(desc[0]), int(desc[1])
    for r in range(rows):
        s, t, c = (int(v) for v in meta[r])
        for p in range(scratch):
            if not (p * 64 < c or p == 0):
                continue
            kb = np.zeros((64, 128), np.uint8)
            sb = np.zeros(64, np.float32)
            for o in range(64):
                i = p * 64 + o
                if i < c:
                    lg = i if i < s else t + i - s
                    lp = lg // 64
                    up = lp if lp < sp else sp + lp - tp
                    kb[o] = uk[up, lg % 64]
                    sb[o] = us[up, lg % 64]
            out[r * scratch + p] = np.concatenate([kb.reshape(-1), sb.view(np.uint8)])
    return out


def union_tables(lens, end, takes, selected, desc, cap, max_take, scratch, fp, S, W, shared):
    """experiments/fine_pool_shared_20261021/kernels.py:13-35: (ft [rows, fp],
    dg_lens [rows], canonical lens [rows])."""
    rows = len(lens)
    ft = np.zeros((rows, fp), np.int32)
    dg = np.zeros(rows, np.int32)
    cl = np.zeros(rows, np.int32)
    for r in range(rows):
        n, take = int(lens[r]), int(takes[r])
        s, t, c = union_bounds(n, end, S, W)
        if shared:
            sp = (s + 63) // 64
            tp = max(sp, t // 64)
            ep = (n + 63) // 64
            gsp, gtp = int(desc[0]), int(desc[1])
            pages = sp + max(ep - tp, 0)
            span = sp * 64 + n - tp * 64 if ep > tp else n
        else:
            pages, span = (c + 63) // 64, c
        for j in range(fp):
            if j < take:
                ft[r, j] = selected[r, j] if j < max_take else 0
            else:
                k = j - take
                if shared:
                    page = cap + k if k < sp else cap + gsp + tp - gtp + k - sp
                else:
                    page = cap + r * scratch + k
                ft[r, j] = page if 0 <= k < pages else 0
        dg[r] = max(take * 64 + span, 1)
        cl[r] = take * 64 + c
    return ft, dg, cl


def union_normalize(raw, lens, end, takes, selected, members, max_take, width, S, W, shared):
    """kernels.py:38-59: scores in canonical candidate order (history members,
    sink, tail), -inf where masked; raw [rows, >= span]."""
    rows = len(lens)
    out = np.full((rows, width), NEG_INF, np.float32)
    for r in range(rows):
        n, take = int(lens[r]), int(takes[r])
        s, t, c = union_bounds(n, end, S, W)
        hist = take * 64
        sp = (s + 63) // 64
        tp = max(sp, t // 64)
        for j in range(width):
            if j < hist:
                page = int(selected[r, j // 64])
                m = int(members[page, j % 64])
                ok = s <= m < t and m < n and m < end
                src = j
            else:
                x = j - hist
                ok = x < c
                lg = x if x < s else t + x - s
                src = hist + (lg if lg < sp * 64 else sp * 64 + lg - tp * 64) if shared else j
            if ok:
                out[r, j] = raw[r, src]
    return out


def union_map_topk(ids, values, lens, end, takes, selected, members, nt, S, W):
    """kernels.py:62-76: (logical, slots) [rows, top] of Top-K candidate ids."""
    rows, top = ids.shape
    logical = np.full((rows, top), -1, np.int32)
    slots = np.full((rows, top), -1, np.int32)
    for r in range(rows):
        n, take = int(lens[r]), int(takes[r])
        s, t, c = union_bounds(n, end, S, W)
        for i in range(top):
            rank = int(ids[r, i])
            if rank < take * 64:
                lg = int(members[int(selected[r, rank // 64]), rank % 64])
            else:
                x = rank - take * 64
                lg = x if x < s else t + x - s
            if values[r, i] != NEG_INF and 0 <= lg < n:
                logical[r, i] = lg
                slots[r, i] = int(nt[lg // 64]) * 64 + lg % 64
    return logical, slots



# ------------------------------------------------- attention consumer
def decode_attention(q, k, v, scale, seqlens=None):
    """sglang/srt/layers/attention/v1_native/backend.py:306-315
    (flash_attn_with_kvcache(q[:, None], kg, vg, causal=False, softmax_scale)),
    one query position per row: q [B, Hq, D], k / v [B, S, Hkv, D] (float
    values of the bf16 inputs); out[b, h] = softmax over the first n_b keys of
    scale * q . k, times v, in float64 (zeros for a row without keys)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, D = q.shape
    S, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D))
    for b in range(B):
        n = S if seqlens is None else min(max(int(seqlens[b]), 0), S)
        if n == 0:
            continue
        for h in range(Hq):
            s = scale * (k[b, :n, h // G] @ q[b, h])
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ v[b, :n, h // G]
    return out


def union_normalize_split(hist, uni, lens, end, takes, selected, members, desc, width, S, W):
    """Canonical scores from split scoring: history candidate j of row r reads
    hist[r, page * 64 + slot] (page = selected[r, j // 64]); tail candidate
    reads uni[r, up * 64 + slot] in union coordinates (up = lp < sp ? lp :
    sp + lp - tp, union.py:33-35); masks as union_normalize."""
    rows = len(lens)
    out = np.full((rows, width), NEG_INF, np.float32)
    sp, tp = int(desc[0]), int(desc[1])
    for r in range(rows):
        n, take = int(lens[r]), int(takes[r])
        s, t, c = union_bounds(n, end, S, W)
        for j in range(width):
            if j < take * 64:
                page = int(selected[r, j // 64])
                m = int(members[page, j % 64])
                if s <= m < t and m < n and m < end:
                    out[r, j] = hist[r, page * 64 + j % 64]
            elif j - take * 64 < c:
                x = j - take * 64
                lg = x if x < s else t + x - s
                lp = lg // 64
                up = lp if lp < sp else sp + lp - tp
                out[r, j] = uni[r, up * 64 + lg % 64]
    return out

