"""GPU parity at the shapes of the five benchmark configurations.

Reduced sizes run against the oracle and compare bit-exactly: full slot-order
exports, returned rows, evicted records (as multisets) and sizes.

At the full sizes the oracle would have to hold the whole table on the host,
so those runs check properties that hold at any size instead.  Every value
row there is a function of its key (`key_rows`), so a row that lands in the
wrong slot, is read from the wrong slot or is torn shows up without a host
copy of the table; keys are MurmurHash3 fmix64 of counters, a bijection, so a
key's counter (and with it the batch that inserted it) is recovered exactly.

The config-5 full-size run allocates 48 GiB of pinned host memory.
"""
import gc

import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, records_equal
from helpers import (RESERVED_MASK, murmur3_np, scramble30, uniform_keys,
                     uniform_keys_fast, zipf_ranks)

pytestmark = pytest.mark.gpu

M1_INV = np.uint64(pow(0xff51afd7ed558ccd, -1, 1 << 64))
M2_INV = np.uint64(pow(0xc4ceb9fe1a85ec53, -1, 1 << 64))


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


# -- full-size helpers --------------------------------------------------------

def _torch():
    import torch
    return torch


def counter_keys(start, n):
    """fmix64(start .. start+n-1): distinct keys; reserved ones dropped."""
    k = murmur3_np(np.arange(start, start + n, dtype=np.uint64))
    return k[(k & RESERVED_MASK) != RESERVED_MASK]


def key_counters(k):
    """Inverse of fmix64 (x ^= x >> 33 is its own inverse; the multiplies
    are undone by their inverses mod 2^64)."""
    x = np.asarray(k, np.uint64).copy()
    with np.errstate(over="ignore"):
        x ^= x >> np.uint64(33)
        x *= M2_INV
        x ^= x >> np.uint64(33)
        x *= M1_INV
        x ^= x >> np.uint64(33)
    return x


def key_rows(keys, dim):
    """fp32 row of each key (int64 cuda tensor): column j holds bits 40..59
    of key*(2j+1) (exact in fp32, being below 2^24)."""
    torch = _torch()
    j = torch.arange(dim, device=keys.device, dtype=torch.int64) * 2 + 1
    return ((keys[:, None] * j[None, :]) >> 40).bitwise_and_(0xFFFFF).to(torch.float32)


def dev(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int64)).cuda()


def host_u64(t):
    return t.cpu().numpy().view(np.uint64)


def new_table(strategy, cap, dim, max_cap=None, max_hbm=None):
    import hkv_amd
    t = hkv_amd.HashTable("u64", "f32", strategy)
    t.init(hkv_amd.HashTableOptions(
        init_capacity=cap, max_capacity=max_cap or cap,
        max_hbm_for_vectors=(max_cap or cap) * dim * 4 if max_hbm is None else max_hbm,
        dim=dim))
    return t


def export_all(t, dim, chunk=1 << 22, on_device=False, row_of=None):
    """Keys and scores of the whole table (slot order), in `chunk`-slot
    export_batch calls, as host uint64 arrays (or int64 cuda tensors); also
    counts exported rows that differ from row_of(keys) (default key_rows)."""
    torch = _torch()
    if row_of is None:
        row_of = lambda k: key_rows(k, dim)  # noqa: E731
    ks = torch.empty(chunk, dtype=torch.int64, device="cuda")
    vs = torch.empty((chunk, dim), dtype=torch.float32, device="cuda")
    ss = torch.empty(chunk, dtype=torch.int64, device="cuda")
    out_k, out_s, bad = [], [], 0
    for off in range(0, t.capacity(), chunk):
        c = t.export_batch(chunk, off, ks, vs, ss)
        if c:
            bad += int((vs[:c] != row_of(ks[:c])).any(dim=1).sum().item())
            if on_device:
                out_k.append(ks[:c].clone())
                out_s.append(ss[:c].clone())
            else:
                out_k.append(host_u64(ks[:c]))
                out_s.append(host_u64(ss[:c]))
    del ks, vs, ss
    if on_device:
        return torch.cat(out_k), torch.cat(out_s), bad
    return np.concatenate(out_k), np.concatenate(out_s), bad


@pytest.fixture(autouse=True)
def _free_device_memory():
    yield
    gc.collect()
    _torch().cuda.empty_cache()


# -- config 2: kLru, capacity 2^26, dim 64 ------------------------------------

def test_c2_shape_lru_fill_to_full():
    """Reduced config 2 (capacity 2^20, dim 64, 2^14-key batches, one clock
    per batch): states at load factors 0.5, 0.75 and 1.0, finds at 100% and
    0% hit, then a batch where every key evicts."""
    rng = np.random.default_rng(201)
    cap, dim, B = 1 << 20, 64, 1 << 14
    p = Pair(cap, dim=dim, strategy=O.LRU, oracle_threads=8)
    resident = []
    b = 0
    for target in (0.5, 0.75, 1.0):
        while p.g.load_factor() < target:
            ks = uniform_keys_fast(rng, B)
            p.insert_or_assign(ks, rand_vals(rng, B, dim), clock=1000 + b)
            resident.append(ks)
            b += 1
        p.assert_same_state()
        allk = np.concatenate(resident)
        q = np.concatenate([rng.choice(allk, B // 2, replace=False),
                            uniform_keys_fast(rng, B // 2)])
        rng.shuffle(q)
        p.assert_same_find(q, fill=5)
    ks = uniform_keys_fast(rng, B)
    p.insert_or_assign(ks, rand_vals(rng, B, dim), clock=1000 + b)
    p.assert_same_state()
    assert p.g.size() == cap
    assert p.assert_same_find(ks).all()


def test_c2_full_size_lru_properties():
    """Config 2 at full size (kLru, 2^26 slots, dim 64, 2^20-key batches):
    fill to 0.5, every key found with its row and its batch's clock, misses
    found nowhere, export = inserted set, erase 10%, fill to 1.0."""
    torch = _torch()
    cap, dim, B = 1 << 26, 64, 1 << 20
    t = new_table(O.LRU, cap, dim)
    batches = []
    for b in range(cap // 2 // B):
        k = counter_keys(b * B, B)
        kd = dev(k)
        t.set_lru_clock(1000 + b)
        t.insert_or_assign(k.size, kd, key_rows(kd, dim))
        batches.append(k)
    n_in = sum(k.size for k in batches)
    assert t.size() == n_in
    out = torch.empty((B, dim), dtype=torch.float32, device="cuda")
    fnd = torch.empty(B, dtype=torch.uint8, device="cuda")
    sc = torch.empty(B, dtype=torch.int64, device="cuda")
    for b, k in enumerate(batches):
        kd = dev(k)
        out.fill_(-1.0)
        t.find(k.size, kd, out, fnd, sc)
        assert bool(fnd[:k.size].bool().all())
        assert torch.equal(out[:k.size], key_rows(kd, dim))
        assert bool((sc[:k.size] == 1000 + b).all())
    miss = counter_keys(1 << 40, B)
    md = dev(miss)
    out.fill_(-1.0)
    t.find(miss.size, md, out, fnd, None)
    assert not bool(fnd[:miss.size].bool().any())
    assert bool((out == -1.0).all())
    mk = torch.empty(B, dtype=torch.int64, device="cuda")
    mi = torch.empty(B, dtype=torch.int32, device="cuda")
    ms = torch.empty(1, dtype=torch.int32, device="cuda")
    t.find_missed(miss.size, md, out, mk, mi, ms)
    m = int(ms.item())
    assert m == miss.size
    assert np.array_equal(np.sort(host_u64(mk[:m])), np.sort(miss))
    assert np.array_equal(np.sort(mi[:m].cpu().numpy()), np.arange(m))
    ek, es, bad = export_all(t, dim)
    assert bad == 0 and ek.size == n_in
    ctr = key_counters(ek)
    assert np.array_equal(np.sort(ctr), np.sort(key_counters(np.concatenate(batches))))
    assert np.array_equal(es, 1000 + ctr // np.uint64(B))
    # erase 10%
    rng = np.random.default_rng(202)
    allk = np.concatenate(batches)
    er = allk[rng.choice(allk.size, allk.size // 10, replace=False)]
    for i in range(0, er.size, B):
        t.erase(min(B, er.size - i), dev(er[i:i + B]))
    assert t.size() == n_in - er.size
    q = er[:B]
    t.find(q.size, dev(q), out, fnd, None)
    assert not bool(fnd[:q.size].bool().any())
    # fill to load factor 1.0, then one batch where every key evicts
    b = len(batches)
    while t.size() < t.capacity():
        k = counter_keys(b * B, B)
        kd = dev(k)
        t.set_lru_clock(1000 + b)
        t.insert_or_assign(k.size, kd, key_rows(kd, dim))
        b += 1
        assert b < 200
    last = counter_keys(b * B, B)
    kd = dev(last)
    t.set_lru_clock(1000 + b)
    t.insert_or_assign(last.size, kd, key_rows(kd, dim))
    assert t.size() == cap
    t.find(last.size, kd, out, fnd, sc)
    assert bool(fnd[:last.size].bool().all())
    assert torch.equal(out[:last.size], key_rows(kd, dim))
    ek, es, bad = export_all(t, dim)
    assert bad == 0 and ek.size == cap
    ctr = key_counters(ek)
    assert np.unique(ctr).size == cap and int(ctr.max()) < (b + 1) * B
    assert np.array_equal(es, 1000 + ctr // np.uint64(B))
    erased = np.zeros((b + 1) * B, bool)
    erased[key_counters(er).astype(np.int64)] = True
    assert not erased[ctr.astype(np.int64)].any()


# -- config 3: kEpochLfu, Zipf(1.05) keys, find_or_insert ----------------------

def test_c3_shape_zipf_epoch_lfu():
    """Reduced config 3 (capacity 2^17, dim 32, 2^13-key Zipf batches,
    epoch + 1 every 10 batches, find_or_insert with duplicates, score
    increment 1): the table saturates and evicts; returned rows and states
    match the oracle."""
    rng = np.random.default_rng(203)
    cap, dim, B = 1 << 17, 32, 1 << 13
    p = Pair(cap, dim=dim, strategy=O.EPOCH_LFU)
    ones = np.ones(B, np.uint64)
    for b in range(60):
        p.set_global_epoch(b // 10)
        ks = scramble30(zipf_ranks(rng, B, 1.05, 1 << 30))
        ov, gv = p.find_or_insert(ks, rand_vals(rng, B, dim), ones, unique_key=False)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
        if b % 10 == 9:
            p.assert_same_state()
    assert p.g.size() == cap


def test_c3_full_size_zipf_epoch_lfu_properties():
    """Config 3 at full size (kEpochLfu, 2^27 slots, dim 32, 200 batches of
    2^20 Zipf(1.05) keys over 2^30, epoch + 1 every 10 batches).  These
    batches hold about 4e7 distinct keys, so no bucket fills and nothing is
    evicted: then every key seen is stored, with score (epoch of its last
    occurrence << 32) | (its number of occurrences), which is checked for
    every key.  Batch b's input row of a key is its key row with column 0 set
    to b, so the rows that come back tell a copied-out table row (column 0 =
    the batch of the key's first occurrence) from an input left in place."""
    torch = _torch()
    cap, dim, B = 1 << 27, 32, 1 << 20
    t = new_table(O.EPOCH_LFU, cap, dim)
    rng = np.random.default_rng(204)
    count = np.zeros(1 << 30, np.uint32)
    last = np.zeros(1 << 30, np.uint8)
    first = torch.full((1 << 30,), 255, dtype=torch.uint8, device="cuda")
    ones = torch.ones(B, dtype=torch.int64, device="cuda")

    def rows_with(kd, col0):
        r = key_rows(kd, dim)
        r[:, 0] = col0
        return r

    copied_out = 0
    for b in range(200):
        e = b // 10
        t.set_global_epoch(e)
        ks = scramble30(zipf_ranks(rng, B, 1.05, 1 << 30))
        kd = dev(ks)
        v = rows_with(kd, float(b))
        t.find_or_insert(B, kd, v, ones, 0, False)
        fresh = first[kd] == 255
        first[kd[fresh]] = b
        fb = first[kd].to(torch.float32)
        assert torch.equal(v, rows_with(kd, fb)), b
        copied_out += int((fb != b).sum().item())
        u, c = np.unique(ks, return_counts=True)
        count[u] += c.astype(np.uint32)
        last[u] = e
    assert copied_out > 20 * B  # many occurrences hit rows of earlier batches
    seen = np.flatnonzero(count)
    assert t.size() == seen.size
    ek, es, bad = export_all(t, dim, row_of=lambda k: rows_with(k, first[k].to(torch.float32)))
    assert bad == 0
    o = np.argsort(ek)
    assert np.array_equal(ek[o], seen.astype(np.uint64))
    want = (last[seen].astype(np.uint64) << np.uint64(32)) | count[seen].astype(np.uint64)
    assert np.array_equal(es[o], want)


# -- config 4: kLfu, dim 128, full table: insert_and_evict, accum, scores -----



def test_c4_shape_lfu_evict_accum_scores():
    """Reduced config 4 (kLfu, capacity 2^15, dim 128): prefill to load factor
    1.0 with uint32 scores, then insert_and_evict, accum_or_assign (deltas in
    [-0.01, 0.01], accumulate for resident keys, assign for new ones) and
    assign_scores on 50% new / 50% resident batches."""
    rng = np.random.default_rng(205)
    cap, dim, B = 1 << 15, 128, 1 << 12
    p = Pair(cap, dim=dim, strategy=O.LFU)
    while p.g.load_factor() < 1.0:
        ks = uniform_keys_fast(rng, B)
        p.insert_or_assign(ks, rand_vals(rng, B, dim),
                           rng.integers(0, 1 << 32, B, dtype=np.uint64))
    p.assert_same_state()

    def mixed():
        (res, _, _), _ = p.export()
        q = np.concatenate([rng.choice(res, B // 2, replace=False),
                            uniform_keys(rng, B // 2, exclude=res)])
        flags = np.concatenate([np.ones(B // 2, np.uint8), np.zeros(B // 2, np.uint8)])
        o = rng.permutation(B)
        return q[o], flags[o]

    for r in range(3):
        q, _ = mixed()
        o, g = p.insert_and_evict(q, rand_vals(rng, B, dim),
                                  rng.integers(0, 1 << 32, B, dtype=np.uint64))
        assert g[0].size >= B // 2
        records_equal(o, g)
        p.assert_same_state()
        q, flags = mixed()
        flags[:64] ^= 1  # a few mismatched flags: no-ops
        p.accum_or_assign(q, rng.uniform(-0.01, 0.01, (B, dim)).astype(np.float32),
                          flags, rng.integers(0, 1 << 32, B, dtype=np.uint64))
        p.assert_same_state()
        q, _ = mixed()
        p.assign_scores(q, rng.integers(0, 1 << 32, B, dtype=np.uint64))
        p.assert_same_state()
    assert p.g.size() == cap


def test_c4_full_size_lfu_properties():
    """Config 4 at full size (kLfu, 2^26 slots, dim 128, prefilled to load
    factor 1.0 with uint32 scores).  insert_and_evict of 2^19 resident keys
    followed by 2^19 new ones: the resident keys hit (score += input) and
    each new key evicts exactly one key, so (table before) + (new keys) =
    (table after) + (evicted records) as disjoint unions, and evicted rows and
    scores are the victims'.  accum_or_assign then adds fp32 deltas to
    resident rows bit-exactly and assigns new keys; assign_scores adds input
    scores to found keys."""
    torch = _torch()
    cap, dim, B, H = 1 << 26, 128, 1 << 20, 1 << 19
    t = new_table(O.LFU, cap, dim)
    rng = np.random.default_rng(206)
    ctr = 0
    while t.size() < t.capacity():
        k = counter_keys(ctr, B)
        ctr += B
        kd = dev(k)
        t.insert_or_assign(k.size, kd, key_rows(kd, dim),
                           dev(rng.integers(0, 1 << 32, k.size, dtype=np.uint64)))
        assert ctr < 200 * B
    k0, s0, bad = export_all(t, dim, on_device=True)
    assert bad == 0 and k0.numel() == cap
    res_i = torch.from_numpy(rng.choice(cap, H, replace=False)).cuda()
    fresh = dev(counter_keys(ctr, H))
    ctr += H
    qd = torch.cat([k0[res_i], fresh])
    n = qd.numel()
    qs = dev(rng.integers(0, 1 << 32, n, dtype=np.uint64))
    ek = torch.empty(n, dtype=torch.int64, device="cuda")
    ev = torch.empty((n, dim), dtype=torch.float32, device="cuda")
    es = torch.empty(n, dtype=torch.int64, device="cuda")
    c = t.insert_and_evict(n, qd, key_rows(qd, dim), qs, ek, ev, es)
    assert c == fresh.numel()
    assert torch.equal(ev[:c], key_rows(ek[:c], dim))
    k1, s1, bad = export_all(t, dim, on_device=True)
    assert bad == 0 and k1.numel() == cap
    lhs = torch.sort(torch.cat([k0, fresh])).values
    rhs = torch.sort(torch.cat([k1, ek[:c]])).values
    assert torch.equal(lhs, rhs)
    # scores: resident batch keys gained their input; others kept theirs
    want = s0.clone()
    want[res_i] += qs[:H]
    allk, oa = torch.sort(torch.cat([k0, fresh]))
    alls = torch.cat([want, qs[H:]])[oa]
    for keys, scores in ((k1, s1), (ek[:c], es[:c])):
        idx = torch.searchsorted(allk, keys)
        assert torch.equal(allk[idx], keys)
        assert torch.equal(alls[idx], scores)
    k1 = host_u64(k1)
    del k0, s0, s1, lhs, rhs, allk, alls, want, ev, oa

    # accum_or_assign: 2^19 resident (accumulate) + 2^19 new (assign), with
    # 1024 of each given the other flag (no-ops).
    res_i = rng.choice(k1.size, H, replace=False)
    res = k1[res_i]
    fresh = counter_keys(ctr, H)
    ctr += H
    q = np.concatenate([res, fresh])
    flags = np.concatenate([np.ones(H, np.uint8), np.zeros(H, np.uint8)])
    flags[:1024] = 0
    flags[H:H + 1024] = 1
    qd = dev(q)
    fd = torch.from_numpy(flags).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(206)
    deltas = torch.rand((q.size, dim), device="cuda", generator=gen) * 0.02 - 0.01
    out = torch.empty((q.size, dim), dtype=torch.float32, device="cuda")
    fnd = torch.empty(q.size, dtype=torch.uint8, device="cuda")
    t.find(q.size, qd, out, fnd, None)
    rows0 = out.clone()
    t.accum_or_assign(q.size, qd, deltas, fd,
                      dev(rng.integers(0, 1 << 32, q.size, dtype=np.uint64)))
    assert t.size() == cap
    out.fill_(-7.0)
    t.find(q.size, qd, out, fnd, None)
    f = fnd.bool()
    acc = f.clone()
    acc[H:] = False
    acc[:1024] = False
    assert torch.equal(out[acc], rows0[acc] + deltas[acc])
    assert bool(f[1024:H].float().mean() > 0.9)  # resident keys stay unless evicted
    assert torch.equal(out[:1024][f[:1024]], rows0[:1024][f[:1024]])
    assert not bool(f[H:H + 1024].any())
    newk = f.clone()
    newk[:H + 1024] = False
    assert torch.equal(out[newk], deltas[newk])
    # Only the inserting keys (new, flag clear: batch indices H + 1024 on)
    # evict, Lfu never refuses them, and a key can only be evicted by a later
    # key of its bucket: so the last inserting key of every bucket is present.
    ins = q[H + 1024:]
    bk = (murmur3_np(ins) & np.uint64(cap - 1)) >> np.uint64(7)
    _, last_rev = np.unique(bk[::-1], return_index=True)
    last_ins = ins.size - 1 - last_rev
    f_ins = f[H + 1024:].cpu().numpy()
    assert f_ins[last_ins].all()
    assert int(f_ins.sum()) >= last_ins.size

    # assign_scores: found keys gain the input score; absent keys stay absent
    sc0 = torch.empty(q.size, dtype=torch.int64, device="cuda")
    t.find(q.size, qd, out, fnd, sc0)
    f0 = fnd.bool().clone()
    inc = torch.from_numpy(rng.integers(0, 1 << 32, q.size, dtype=np.uint64)
                           .view(np.int64)).cuda()
    t.assign_scores(q.size, qd, inc)
    sc1 = torch.empty(q.size, dtype=torch.int64, device="cuda")
    t.find(q.size, qd, out, fnd, sc1)
    assert torch.equal(fnd.bool(), f0)
    assert torch.equal(sc1[f0], sc0[f0] + inc[f0])
    assert t.size() == cap


# -- config 5: kCustomized, hybrid HBM/host rows, reserve, chunked export ------

def test_c5_shape_hybrid_reserve_export():
    """Reduced config 5 (kCustomized, init 2^15 growing to 2^16, dim 64,
    a quarter of the grown table's rows in HBM and the rest in pinned host
    memory): mixed find / insert_or_assign batches until auto-growth
    doubles the capacity, then export_batch over the whole table in chunks."""
    rng = np.random.default_rng(207)
    init, mx, dim, B = 1 << 15, 1 << 16, 64, 1 << 12
    p = Pair(init, mx, dim=dim, strategy=O.CUSTOMIZED, max_hbm=(mx * dim * 4) // 4)
    assert not p.g.is_pure_hbm_mode()
    resident = np.empty(0, np.uint64)
    grown = 0
    for b in range(16):
        if resident.size:
            q = np.concatenate([rng.choice(resident, B // 2, replace=False),
                                uniform_keys_fast(rng, B // 2)])
            p.assert_same_find(q, fill=2)
        ks = uniform_keys_fast(rng, B)
        p.insert_or_assign(ks, rand_vals(rng, B, dim),
                           rng.integers(0, 2**64 - 1, B, dtype=np.uint64))
        resident = np.concatenate([resident, ks])
        if p.g.capacity() == mx and not grown:
            grown = b
            p.assert_same_state()
    assert grown and p.g.capacity() == mx
    for off in range(0, mx, 1 << 13):
        (ok, ov, os_), (gk, gv, gs) = p.export(1 << 13, off)
        np.testing.assert_array_equal(gk, ok)
        np.testing.assert_array_equal(gs, os_)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    p.assert_same_state()
    # explicit reserve from a high load factor
    q = Pair(init, mx, dim=dim, strategy=O.CUSTOMIZED, max_hbm=(mx * dim * 4) // 4,
             max_load_factor=1.0)
    while q.g.load_factor() < 0.9:
        ks = uniform_keys_fast(rng, B)
        q.insert_or_assign(ks, rand_vals(rng, B, dim),
                           rng.integers(0, 2**64 - 1, B, dtype=np.uint64))
    q.reserve(mx)
    assert q.g.capacity() == mx
    q.assert_same_state()


def test_c5_full_size_hybrid_properties():
    """Config 5 at full size (kCustomized, init 2^27 growing to 2^28, dim 64,
    max_hbm_for_vectors 16 GiB, so after growth 3/4 of the rows are pinned
    host memory): mixed find / insert_or_assign batches of 2^20 keys until
    auto-growth, then export_batch over the whole table in 2^22-slot chunks.
    Scores are the keys' counters, rows key_rows(key)."""
    torch = _torch()
    init, mx, dim, B = 1 << 27, 1 << 28, 64, 1 << 20
    t = new_table(O.CUSTOMIZED, init, dim, max_cap=mx, max_hbm=16 << 30)
    assert not t.is_pure_hbm_mode()
    out = torch.empty((B, dim), dtype=torch.float32, device="cuda")
    fnd = torch.empty(B, dtype=torch.uint8, device="cuda")
    sc = torch.empty(B, dtype=torch.int64, device="cuda")
    b = 0
    rng = np.random.default_rng(208)
    while t.capacity() < mx or b < 72:
        if b:
            q = np.concatenate([counter_keys(rng.integers(0, b) * B + 7, B // 2),
                                counter_keys((1 << 40) + b * B, B // 2)])
            qd = dev(q)
            out.fill_(-1.0)
            t.find(q.size, qd, out, fnd, sc)
            f = fnd[:q.size].bool()
            assert bool(f[:B // 2].all()) and not bool(f[B // 2:].any())
            assert torch.equal(out[:B // 2], key_rows(qd[:B // 2], dim))
            assert bool((out[B // 2:q.size] == -1.0).all())
            assert np.array_equal(host_u64(sc[:B // 2]), key_counters(q[:B // 2]))
        k = counter_keys(b * B, B)
        kd = dev(k)
        t.insert_or_assign(k.size, kd, key_rows(kd, dim), dev(key_counters(k)))
        b += 1
        assert b < 100
    assert t.capacity() == mx
    assert t.size() == sum(counter_keys(i * B, B).size for i in range(b))
    ek, es, bad = export_all(t, dim)
    assert bad == 0
    assert np.array_equal(es, key_counters(ek))
    assert np.array_equal(np.sort(es), np.sort(np.concatenate(
        [key_counters(counter_keys(i * B, B)) for i in range(b)])))
