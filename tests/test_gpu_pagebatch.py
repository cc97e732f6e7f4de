"""GPU parity of the batched page manager (insert = match_pages -> allocate ->
publish request after request, release in list order) and of the device-wide
pair sort, against the CPU oracle: tables, refs, free stack, count, pool bytes
and keys bit-exact.  All calls go through the C ABI of libv1idx.so."""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O

pytestmark = pytest.mark.gpu

PP = pkg("pagepool")
W = pkg("workloads")


def T(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def H(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_pool(dev, pool, pool_keys, refs, free, count):
    p = PP.PagePool(len(refs), pool.shape[1], dev)
    p.pool.copy_(T(pool, dev))
    p.keys.copy_(T(pool_keys, dev))
    p.refs.copy_(T(refs, dev))
    p.free.copy_(T(free, dev))
    p.count.fill_(int(count))
    return p


def state(p):
    return H(p.pool), H(p.keys), H(p.refs), H(p.free), int(H(p.count)[0])


def assert_state(p, pool, pool_keys, refs, free, count):
    gp, gk, gr, gf, gc = state(p)
    assert gc == count
    assert np.array_equal(gr, refs)
    assert np.array_equal(gf[:count], free[:count])
    assert np.array_equal(gp, pool)
    live = refs > 0
    assert np.array_equal(gk[live], pool_keys[live])


# ------------------------------------------------------------------ sort
@pytest.mark.parametrize("n,distinct", [(1, 1), (4095, 7), (4097, 4097), (200003, 50), (131072, 1 << 40)])
def test_sort_pairs_u64_stable(dev, n, distinct):
    g = np.random.default_rng(n)
    keys = g.integers(-(distinct // 2) - 1, distinct // 2 + 1, n).astype(np.int64) * 0x9E3779B97F4A7C1
    vals = np.arange(n, dtype=np.int32)
    ko, vo = PP.sort_pairs_u64(T(keys, dev), T(vals, dev))
    order = np.argsort(keys.view(np.uint64), kind="stable")
    assert np.array_equal(H(vo), vals[order]) and np.array_equal(H(ko), keys[order])


# -------------------------------------------------------------- insert
def test_page_lifecycle_kat_batched(dev, kats):
    kat = kats["page_lifecycle"]
    cap = kat["capacity"]
    p = PP.PagePool(cap, 8448, dev)
    tmp = torch.arange(16, device=dev, dtype=torch.uint8)[:, None].expand(16, 8448).contiguous()
    keys = torch.arange(16, device=dev, dtype=torch.int64) * 1000003
    req = torch.zeros(16, device=dev, dtype=torch.int32)
    t0 = p.insert(keys, tmp, req)
    assert H(t0).tolist() == kat["first_table"] and int(H(p.count)[0]) == kat["count_after_first"]
    assert bool((p.refs == kat["refs_after_first"]).all()) and torch.equal(p.pool[t0.long()], tmp)
    t1 = p.insert(keys, tmp, req)
    assert torch.equal(t1, t0) and bool((p.refs == kat["refs_after_second"]).all())
    p.release(t0)
    assert int(H(p.count)[0]) == 0 and bool((p.refs == kat["refs_after_release_a"]).all())
    p.release(t1)
    assert int(H(p.count)[0]) == kat["count_after_release_b"]
    assert sorted(H(p.free).tolist()) == list(range(16)) and p.status() == 0


def _prelive(g, cap, keys, tmp, n_live=40):
    pool = g.integers(0, 256, (cap, tmp.shape[1]), dtype=np.uint8)
    pool_keys = g.integers(-2**62, 2**62, cap)
    refs = np.zeros(cap, np.int32)
    pick = g.choice(len(keys), n_live // 2, replace=False)
    live = g.choice(cap, n_live, replace=False)
    pool[live[:n_live // 2]] = tmp[pick]
    pool_keys[live[:n_live // 2]] = keys[pick]
    pool_keys[live[n_live // 2:n_live // 2 + n_live // 4]] = keys[pick[:n_live // 4]]  # live collisions
    refs[live] = g.integers(1, 4, n_live)
    free_pages = np.setdiff1d(np.arange(cap), live)
    free = np.concatenate([g.permutation(free_pages), np.full(n_live, -7)]).astype(np.int32)
    return pool, pool_keys, refs, free, len(free_pages)


@pytest.mark.parametrize("seed,page_bytes,collide", [(1, 16, 0), (2, 656, 6), (3, 8448, 3), (4, 41984, 4)])
def test_page_insert_then_release_vs_oracle(dev, seed, page_bytes, collide):
    cap = 3000
    wl = W.config2(seed=seed, requests=160, max_pages=24, capacity=cap, collide=collide)
    a = wl.arrays
    keys, req = a["keys"], a["req"]
    tmp = W.config2_payload(wl, page_bytes)[a["draw"]]
    g = np.random.default_rng(seed)
    st = _prelive(g, cap, keys, tmp)
    print(f"insert seed={seed} page_bytes={page_bytes} entries={len(keys)}", flush=True)
    p = make_pool(dev, *st)
    # two batches: the second sees the first's pages (live or released)
    half = int(np.searchsorted(req, 80))
    t_a = H(p.insert(T(keys[:half], dev), T(tmp[:half], dev), T(req[:half], dev)))
    exp_a = O.page_insert_batch(*st, keys[:half], tmp[:half], req[:half])
    assert np.array_equal(t_a, exp_a[0])
    assert_state(p, *exp_a[1:])
    rel = W.config2_release_list(wl, np.concatenate([t_a, np.zeros(len(keys) - half, np.int32)]))
    rel = rel[:np.count_nonzero(wl.arrays["released"][req[:half]])]
    p.release(T(rel, dev))
    refs_r, free_r, count_r = O.page_release_batch(rel, exp_a[3], exp_a[4], exp_a[5])
    assert_state(p, exp_a[1], exp_a[2], refs_r, free_r, count_r)
    t_b = H(p.insert(T(keys[half:], dev), T(tmp[half:], dev), T(req[half:], dev)))
    exp_b = O.page_insert_batch(exp_a[1], exp_a[2], refs_r, free_r, count_r, keys[half:], tmp[half:], req[half:])
    assert np.array_equal(t_b, exp_b[0])
    assert_state(p, *exp_b[1:])
    assert p.status() == 0


def test_page_insert_collision_classes(dev):
    """One key, many byte contents across requests: the one-wave resolution of
    colliding entries against live pages and earlier entries."""
    g = np.random.default_rng(11)
    cap, n = 1024, 700
    req = np.sort(g.integers(0, 60, n)).astype(np.int32)
    content = g.integers(0, 25, n)
    tmp = np.repeat(content[:, None].astype(np.uint8), 48, axis=1)
    tmp[:, 5] = 200
    keys = np.where(g.random(n) < 0.7, 77, g.integers(0, 3, n)).astype(np.int64)
    pool = np.zeros((cap, 48), np.uint8)
    pool_keys = np.zeros(cap, np.int64)
    refs = np.zeros(cap, np.int32)
    for j, (page, c) in enumerate([(900, 3), (17, 5), (400, 3), (2, 24)]):
        pool[page] = c
        pool[page, 5] = 200
        pool_keys[page] = 77
        refs[page] = 1
    free = np.setdiff1d(np.arange(cap), [900, 17, 400, 2]).astype(np.int32)
    free = np.concatenate([free, np.zeros(4, np.int32)])
    st = (pool, pool_keys, refs, free, cap - 4)
    p = make_pool(dev, *st)
    t = H(p.insert(T(keys, dev), T(tmp, dev), T(req, dev)))
    exp = O.page_insert_batch(*st, keys, tmp, req)
    assert np.array_equal(t, exp[0])
    assert_state(p, *exp[1:])
    assert p.status() == 0


def test_page_insert_all_ones_key_and_dense_keys(dev):
    """The key -1 (all ones: the hash table's free marker) and a batch whose
    keys all fall in one small range (long probe chains)."""
    g = np.random.default_rng(12)
    cap, n = 512, 900
    req = np.sort(g.integers(0, 40, n)).astype(np.int32)
    keys = np.where(g.random(n) < 0.3, -1, g.integers(0, 40, n)).astype(np.int64)
    tmp = np.zeros((n, 32), np.uint8)
    tmp[:, 0] = (keys % 7).astype(np.uint8)
    tmp[:, 1] = g.integers(0, 2, n)  # two byte contents per key: collisions
    pool = np.zeros((cap, 32), np.uint8)
    pool_keys = np.zeros(cap, np.int64)
    refs = np.zeros(cap, np.int32)
    pool_keys[[3, 9]] = -1
    pool[9, 1] = 1
    pool[9, 0] = (-1 % 7)
    refs[[3, 9]] = 2
    free = np.concatenate([np.setdiff1d(np.arange(cap), [3, 9]), [0, 0]]).astype(np.int32)
    st = (pool, pool_keys, refs, free, cap - 2)
    p = make_pool(dev, *st)
    t = H(p.insert(T(keys, dev), T(tmp, dev), T(req, dev)))
    exp = O.page_insert_batch(*st, keys, tmp, req)
    assert np.array_equal(t, exp[0])
    assert_state(p, *exp[1:])
    assert p.status() == 0


def test_page_insert_failures_leave_state(dev):
    g = np.random.default_rng(5)
    cap = 64
    tmp = g.integers(0, 256, (80, 32), dtype=np.uint8)
    keys = np.arange(80, dtype=np.int64)
    req = np.repeat(np.arange(10, dtype=np.int32), 8)
    st = (np.zeros((cap, 32), np.uint8), np.zeros(cap, np.int64), np.zeros(cap, np.int32),
          np.arange(cap, dtype=np.int32), cap)
    p = make_pool(dev, *st)
    table = torch.full((80,), -5, device=dev, dtype=torch.int32)
    p.insert(T(keys, dev), T(tmp, dev), T(req, dev), table)
    assert p.status() == PP.STATUS_EXHAUSTED and bool((table == -5).all())
    assert_state(p, *st[:4], cap)
    bad = req.copy()
    bad[10], bad[11] = 3, 0
    p.insert(T(keys[:40], dev), T(tmp[:40], dev), T(bad[:40], dev))
    assert p.status() & PP.STATUS_BAD_ORDER
    assert_state(p, *st[:4], cap)
    with pytest.raises(RuntimeError, match="exhausted"):
        p.insert(T(keys, dev), T(tmp, dev), T(req, dev))
        p.raise_on_status()
    # more colliding entries than one batch resolves
    n = 4200
    tmp2 = np.zeros((n, 16), np.uint8)
    tmp2[:, :4] = np.arange(n, dtype=np.uint32)[:, None].view(np.uint8)
    big = PP.PagePool(8192, 16, dev)
    big.insert(torch.full((n,), 9, device=dev, dtype=torch.int64), T(tmp2, dev),
               torch.zeros(n, device=dev, dtype=torch.int32))
    assert big.status() == PP.STATUS_COLLISIONS and int(H(big.count)[0]) == 8192
    assert int(big.refs.sum()) == 0


def test_page_release_underflow_leaves_state(dev):
    refs = np.int32([2, 1, 1, 0, 0, 0, 0, 0])
    free = np.int32([7, 6, 5, 4, 3, -1, -1, -1])
    p = make_pool(dev, np.zeros((8, 16), np.uint8), np.zeros(8, np.int64), refs, free, 5)
    for bad in ([0, 0, 0], [3], [1, 9], [-1]):
        p.release(T(np.int32(bad), dev))
        assert p.status() == PP.STATUS_UNDERFLOW, bad
        assert np.array_equal(H(p.refs), refs) and int(H(p.count)[0]) == 5
    p.release(T(np.int32([0, 1, 0, 2]), dev))
    assert p.status() == 0 and int(H(p.count)[0]) == 8
    assert H(p.free)[5:8].tolist() == [1, 0, 2] and H(p.refs).tolist() == [0] * 8


# ------------------------------------------------ page management workload
def test_config2_full_batch_vs_oracle(dev):
    """4096 requests, ~132 K entries, 65536-page pool: the equality classes of
    the pages decide every result, so 656-byte pages (one MLA row) give the
    oracle's tables for the full 41984-byte workload too."""
    wl = W.config2(collide=8)
    a = wl.arrays
    cap = wl.params["capacity"]
    tmp = W.config2_payload(wl, 656)[a["draw"]]
    st = (np.zeros((cap, 656), np.uint8), np.zeros(cap, np.int64), np.zeros(cap, np.int32),
          np.arange(cap, dtype=np.int32), cap)
    print(f"config2 entries={len(a['keys'])}", flush=True)
    p = make_pool(dev, *st)
    t = H(p.insert(T(a["keys"], dev), T(tmp, dev), T(a["req"], dev)))
    exp = O.page_insert_batch(*st, a["keys"], tmp, a["req"])
    assert np.array_equal(t, exp[0])
    assert_state(p, *exp[1:])
    rel = W.config2_release_list(wl, t)
    p.release(T(rel, dev))
    refs_r, free_r, count_r = O.page_release_batch(rel, exp[3], exp[4], exp[5])
    assert_state(p, exp[1], exp[2], refs_r, free_r, count_r)
    assert p.status() == 0


def test_config2_full_pages_match_row_tables(dev):
    """Full 41984-byte pages generated on the device: same tables as with
    one-row pages of the same equality classes, and every table page holds its
    entry's bytes."""
    wl = W.config2()
    a = wl.arrays
    cap, pb = wl.params["capacity"], wl.params["page_bytes"]
    gen = torch.Generator(device=dev).manual_seed(2)
    uniq = torch.randint(0, 256, (wl.params["distinct"], pb), generator=gen, device=dev, dtype=torch.uint8)
    draw = T(a["draw"], dev).long()
    tmp = uniq[draw]
    keys, req = T(a["keys"], dev), T(a["req"], dev)
    big = PP.PagePool(cap, pb, dev)
    t_big = big.insert(keys, tmp, req)
    small = PP.PagePool(cap, 16, dev)
    t_small = small.insert(keys, uniq[:, :16][draw].contiguous(), req)
    assert torch.equal(t_big, t_small) and torch.equal(big.refs, small.refs)
    assert torch.equal(big.count, small.count)
    assert torch.equal(big.pool[t_big.long()], tmp)
    assert big.status() == 0 and small.status() == 0


# ------------------------------------------------------ tail staging (rows)
@pytest.mark.parametrize("rows,row_bytes,scratch", [(4, 656, 68), (37, 656, 20), (9, 32, 68)])
def test_stage_tail_rows_vs_oracle(dev, rows, row_bytes, scratch):
    g = np.random.default_rng(rows)
    pages, cap = 300, 50
    native = g.integers(0, 256, (pages, 64 * row_bytes), dtype=np.uint8)
    np_ = 40
    nt = g.integers(0, pages, (rows, np_)).astype(np.int32)
    lens = g.integers(1, np_ * 64 + 1, rows).astype(np.int32)
    lens[:2] = [1100, 64]
    owners = np.where(g.random(rows) < 0.4, 0, np.arange(rows)).astype(np.int32)
    fine = np.full((cap + rows * scratch, 64 * row_bytes), 255, np.uint8)
    exp = fine.copy()
    O.stage_tail_rows(native, nt, lens, exp, cap, scratch, 64, 64, row_bytes, tail_rows=owners)
    f = T(fine, dev)
    PP.stage_tail_rows(T(native, dev), T(nt, dev), T(lens, dev), f, T(owners, dev), cap, scratch)
    assert np.array_equal(H(f), exp)


def test_config2_tail_staging_vs_oracle(dev):
    """128-token tails of 2048 owner requests over the page pool the batch
    insert filled (656-byte rows, 41984-byte pages)."""
    wl = W.config2()
    a = wl.arrays
    cap, pb = wl.params["capacity"], wl.params["page_bytes"]
    pool = PP.PagePool(cap, pb, dev)
    uniq = W.config2_payload(wl, pb)
    tmp = torch.from_numpy(uniq).to(dev)[T(a["draw"], dev).long()]
    table = H(pool.insert(T(a["keys"], dev), tmp, T(a["req"], dev)))
    tails = W.config2_tails(wl, table)
    R = len(a["lens"])
    fine = torch.zeros((cap + R * tails["scratch"], pb), dtype=torch.uint8, device=dev)
    fine[:cap].copy_(pool.pool)
    PP.stage_tail_rows(pool.pool, T(tails["nt"], dev), T(tails["lens"], dev), fine, T(tails["tail_rows"], dev),
                       cap, tails["scratch"])
    got = H(fine[cap:])
    pool_h = H(pool.pool)
    exp = np.zeros((cap + R * tails["scratch"], pb), np.uint8)
    O.stage_tail_rows(pool_h, tails["nt"], tails["lens"], exp, cap, tails["scratch"], 64, 64, 656,
                      tail_rows=tails["tail_rows"])
    assert np.array_equal(got, exp[cap:])
    assert not got.reshape(R // 2, 2, tails["scratch"], pb)[:, 1].any()  # non-owner scratch stays zero
