"""Pins the oracle (host C++ restatement) before anything is compared to it.

Each check is one the reference's own tests or the mathematics fix, chosen so
that a plausible slip (wrong hash constant, wrong probe order, wrong score
functor arithmetic, wrong tie-break) fails at least one of them:

* closed forms: MurmurHash3 fmix64, the empty/reclaim digests, exact
  magic-number modulo for power-of-two and general capacities;
* score-functor known answers from tests/test_score_functor/test_score_functor.cpp;
* end-to-end known answers from tests/test_insert_or_assign.cpp,
  tests/community/merlin_hashtable_test.cpp, tests/test_insert_and_evict.cpp,
  tests/test_find_miss.cpp, tests/test_erase.cpp, tests/test_reserve.cpp;
* invariants: every stored key is found, bucket sizes equal live slots,
  threaded mode equals one thread, digest path equals tile path placement.
"""
import numpy as np
import pytest

import oracle as O
from helpers import keys_in_bucket, murmur3_np, uniform_keys, values_for

MASK64 = (1 << 64) - 1


def fmix64_py(k):
    k ^= k >> 33
    k = (k * 0xff51afd7ed558ccd) & MASK64
    k ^= k >> 33
    k = (k * 0xc4ceb9fe1a85ec53) & MASK64
    k ^= k >> 33
    return k


def test_murmur3_closed_form():
    rng = np.random.default_rng(1)
    ks = [0, 1, 2, MASK64, MASK64 - 1, 1 << 63] + [
        int(x) for x in rng.integers(0, 2**64, 200, dtype=np.uint64)]
    for k in ks:
        assert O.murmur3(k) == fmix64_py(k)
    assert O.murmur3(0) == 0  # fmix64 fixes zero
    np.testing.assert_array_equal(
        murmur3_np(np.array(ks, np.uint64)),
        np.array([fmix64_py(k) for k in ks], np.uint64))


def test_digest_constants():
    # include/types.h:96-106 derive them from the hash of the sentinels.
    L = O.lib()
    assert L.hkvo_empty_digest() == 0x0b
    assert L.hkvo_reclaim_digest() == 0x88
    assert (fmix64_py(MASK64) >> 32) & 0xFF == 0x0b
    assert (fmix64_py(MASK64 - 1) >> 32) & 0xFF == 0x88


@pytest.mark.parametrize("cap", [128, 1 << 20, 1 << 26, 1 << 28, 3 << 20,
                                 10**8, 128 * 1000 + 0, 128 * 7919, 2**40 + 128])
def test_quick_div_exact(cap):
    rng = np.random.default_rng(cap % 1000)
    hs = [0, 1, cap - 1, cap, cap + 1, 2 * cap - 1, MASK64, MASK64 - cap,
          (MASK64 // cap) * cap, (MASK64 // cap) * cap - 1] + [
        int(x) for x in rng.integers(0, 2**64, 2000, dtype=np.uint64)]
    for h in hs:
        assert O.global_idx(h, cap) == h % cap, (h, cap)


# --- score functor known answers (test_score_functor.cpp:162-473) ---------

def test_score_functor_kats():
    L = O.lib()
    d, n, hit, wo = (L.hkvo_score_desired, L.hkvo_score_new,
                     L.hkvo_score_hit, L.hkvo_score_without_missed)
    IGN = O.IGNORED_GLOBAL_EPOCH
    # desired_when_missed
    assert d(O.LRU, 0, 0, IGN, 9876543210) == 9876543210
    assert d(O.LFU, 1, 5, IGN, 0) == MASK64
    assert d(O.EPOCH_LRU, 0, 0, 5, 0x100000000) == (5 << 32) | (
        (0x100000000 >> 20) & 0xFFFFFFFF)
    assert d(O.EPOCH_LFU, 1, 100, 7, 0) == (7 << 32) | 100
    assert d(O.CUSTOMIZED, 1, 12345, IGN, 0) == 12345
    # update: new insert then accumulate
    assert n(O.LRU, 0, 0, 123456, 0) == 123456
    s = n(O.LFU, 1, 999, MASK64, 0)
    assert s == 999
    assert hit(O.LFU, 1, 999, MASK64, s) == 999 + 999
    assert n(O.EPOCH_LRU, 0, 0, (5 << 32) | 123, 0) == (5 << 32) | 123
    s = n(O.EPOCH_LFU, 1, 200, (7 << 32) | 200, 0)
    assert s == (7 << 32) | 200
    assert hit(O.EPOCH_LFU, 1, 200, (7 << 32) | 200, s) == (7 << 32) | 400
    assert n(O.CUSTOMIZED, 1, 88888, 88888, 0) == 88888
    # update_without_missed
    assert wo(O.LRU, 0, 0, IGN, 555555, 7) == 555555
    assert wo(O.LFU, 1, 20, IGN, 0, 10) == 30
    assert wo(O.EPOCH_LRU, 0, 0, 11, 0x200000000, 0) == (11 << 32) | (
        (0x200000000 >> 20) & 0xFFFFFFFF)
    assert wo(O.EPOCH_LFU, 1, 20, 13, 0, (13 << 32) | 50) & 0xFFFFFFFF == 70
    assert wo(O.EPOCH_LFU, 1, 20, 17, 0, (17 << 32) | 60) & 0xFFFFFFFF == 80
    assert wo(O.CUSTOMIZED, 1, 77777, IGN, 0, 5) == 77777
    # EpochLfu saturation: low word never wraps.
    assert hit(O.EPOCH_LFU, 1, 0xFFFFFFFE, (2 << 32) | 0xFFFFFFFE,
               (1 << 32) | 0xFFFFFFFE) == (2 << 32) | 0xFFFFFFFF


# --- end-to-end known answers ----------------------------------------------

def test_fill_to_load_factor_one_takes_166_batches():
    # tests/test_insert_or_assign.cpp:170-228: 1024 consecutive keys per batch
    # into a 128K-slot kLru table reach load factor 1.0 after exactly 166.
    t = O.Oracle(128 * 1024, dim=8, strategy=O.LRU)
    for rnd in range(2):
        t.clear()
        batches = 0
        while t.load_factor() != 1.0:
            ks = np.arange(1024 * batches, 1024 * (batches + 1), dtype=np.uint64)
            t.insert_or_assign(ks, values_for(ks, 8), clock=batches + 1)
            batches += 1
            assert batches <= 166
        assert batches == 166


def test_fill_count_closed_form():
    # The same count from first principles: keys go to buckets by hash; a
    # bucket saturates at 128; count batches until all 1024 are full.
    cnt = np.zeros(1024, np.int64)
    b = 0
    while (cnt < 128).any():
        ks = np.arange(1024 * b, 1024 * (b + 1), dtype=np.uint64)
        bk = (murmur3_np(ks) & np.uint64((1 << 17) - 1)) >> np.uint64(7)
        np.add.at(cnt, bk.astype(np.int64), 1)
        np.minimum(cnt, 128, out=cnt)
        b += 1
    assert b == 166


def test_single_bucket_keeps_128_of_1024():
    # tests/test_insert_or_assign.cpp:230-263
    t = O.Oracle(128, dim=8, strategy=O.LRU)
    ks = np.arange(1024, dtype=np.uint64)
    vals = values_for(ks, 8)
    t.insert_or_assign(ks, vals, clock=7)
    assert t.size() == 128
    got, founds, _ = t.find(ks)
    assert founds.sum() == 128
    np.testing.assert_array_equal(got[founds], vals[founds])


def test_dim27_single_bucket():
    # tests/test_insert_or_assign.cpp:265-305
    t = O.Oracle(128, dim=27, strategy=O.LRU)
    ks = np.arange(1024, dtype=np.uint64)
    vals = values_for(ks, 27)
    t.insert_or_assign(ks, vals, clock=7)
    assert t.size() == 128
    got, founds, _ = t.find(ks)
    assert founds.sum() == 128
    np.testing.assert_array_equal(got[founds], vals[founds])


def _strategy_case(strategy, seed):
    """tests/community/merlin_hashtable_test.cpp:1031-1306, one round."""
    rng = np.random.default_rng(seed)
    B, cap, dim, FREQ = 128, 8 * 128, 4, 1000
    n_test = 128 if strategy == O.CUSTOMIZED else 4
    base = keys_in_bucket(rng, B, cap, 1, lo=0, hi=0x3FFFFFFFFFFFFFFF)
    test = keys_in_bucket(rng, n_test, cap, 1, lo=0x3FFFFFFFFFFFFFFF,
                          hi=0xFFFFFFFFFFFFFFFD)
    lfu = strategy in (O.LFU, O.EPOCH_LFU)
    s_base = (base % np.uint64(FREQ)) if lfu else base.copy()
    s_test = (test % np.uint64(FREQ)) if lfu else test.copy()
    v_base = values_for(base, dim)
    v_test = values_for(test, dim)
    if strategy == O.CUSTOMIZED:
        s_base = np.arange(1000, 1000 + B, dtype=np.uint64)
        s_test = np.arange(1000 + B, 1000 + B + n_test, dtype=np.uint64)
        test[64:] = base[64:n_test]
        v_test[64:] = v_base[64:n_test]
    else:
        test[2], test[3] = base[72], base[73]
        if lfu:
            s_test[2] = base[72] % np.uint64(FREQ)
            s_test[3] = base[73] % np.uint64(FREQ)
        if strategy == O.EPOCH_LFU:
            s_base[71] = np.uint64(0xFFFFFFFF - 1)
            test[1] = base[71]
            s_test[1] = s_base[71]
        start = 1 if strategy == O.EPOCH_LFU else 2
        for i in range(start, n_test):
            v_test[i] = v_base[70 + i]
    return base, s_base, v_base, test, s_test, v_test


def _expected_epochlfu(epoch, orig):
    return (epoch << 32) | (0xFFFFFFFF if orig >= 0xFFFFFFFF else orig & 0xFFFFFFFF)


@pytest.mark.parametrize("strategy", [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU,
                                      O.CUSTOMIZED])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_evict_strategy_basic(strategy, seed):
    base, s_base, v_base, test, s_test, v_test = _strategy_case(strategy, seed)
    t = O.Oracle(8 * 128, dim=4, strategy=strategy)
    sc = None if strategy in (O.LRU, O.EPOCH_LRU) else s_base
    clk1, clk2 = 1_000_000_000 << 20, 2_000_000_000 << 20
    t.set_global_epoch(1)
    t.insert_or_assign(base, v_base, sc, clock=clk1)
    assert t.size() == 128
    k, v, s = t.export_batch(t.capacity())
    assert k.size == 128
    if strategy == O.LFU:
        np.testing.assert_array_equal(s, k % np.uint64(1000))
    elif strategy == O.EPOCH_LFU:
        for kk, ss in zip(k, s):
            orig = int(s_base[71]) if kk == base[71] else int(kk) % 1000
            assert int(ss) == _expected_epochlfu(1, orig)
    elif strategy == O.CUSTOMIZED:
        np.testing.assert_array_equal(np.sort(s), np.arange(1000, 1128))
    elif strategy == O.LRU:
        assert (s == clk1).all()
    else:
        assert (s == ((1 << 32) | ((clk1 >> 20) & 0xFFFFFFFF))).all()
    np.testing.assert_array_equal(v, values_for(k, 4))

    t.set_global_epoch(2)
    sc = None if strategy in (O.LRU, O.EPOCH_LRU) else s_test
    t.insert_or_assign(test, v_test, sc, clock=clk2)
    assert t.size() == 128
    k, v, s = t.export_batch(t.capacity())
    assert k.size == 128
    base_set = set(int(x) for x in base)
    test_set = set(int(x) for x in test)
    if strategy == O.CUSTOMIZED:
        np.testing.assert_array_equal(np.sort(s), np.arange(1128, 1256))
    elif strategy == O.LRU:
        for kk, ss in zip(k, s):
            assert int(ss) == (clk2 if int(kk) in test_set else clk1)
    elif strategy == O.EPOCH_LRU:
        e2 = (2 << 32) | ((clk2 >> 20) & 0xFFFFFFFF)
        e1 = (1 << 32) | ((clk1 >> 20) & 0xFFFFFFFF)
        for kk, ss in zip(k, s):
            assert int(ss) == (e2 if int(kk) in test_set else e1)
    elif strategy == O.LFU:
        for kk, ss in zip(k, s):
            both = int(kk) in base_set and int(kk) in test_set
            assert int(ss) == (int(kk) % 1000) * (2 if both else 1)
    else:
        assert int(base[71]) in set(int(x) for x in k)
        for kk, ss in zip(k, s):
            kb, kt = int(kk) in base_set, int(kk) in test_set
            orig = int(s_base[71]) if kk == base[71] else int(kk) % 1000
            if kb and kt:
                assert int(ss) == _expected_epochlfu(2, orig * 2)
            else:
                assert int(ss) == _expected_epochlfu(2 - int(kb), orig)
    np.testing.assert_array_equal(v, values_for(k, 4))


def test_insert_and_evict_rejects_low_scores():
    # tests/test_insert_and_evict.cpp:679-745 (kCustomized)
    rng = np.random.default_rng(5)
    cap, dim = 4 * 128, 8
    t = O.Oracle(cap, dim=dim, strategy=O.CUSTOMIZED)
    hi = keys_in_bucket(rng, 128, cap, 0, lo=1, hi=10_000_000)
    ek, ev, es = t.insert_and_evict(hi, values_for(hi, dim),
                                    np.arange(500, 628, dtype=np.uint64))
    assert ek.size == 0
    lo = keys_in_bucket(rng, 64, cap, 0, lo=100_000_000, hi=200_000_000)
    lv = values_for(lo, dim)
    ek, ev, es = t.insert_and_evict(lo, lv, np.arange(64, dtype=np.uint64))
    assert ek.size == 64
    np.testing.assert_array_equal(ek, lo)  # batch order
    np.testing.assert_array_equal(ev, lv)
    np.testing.assert_array_equal(es, np.arange(64))
    _, f, _ = t.find(hi)
    assert f.all()
    _, f, _ = t.find(lo)
    assert not f.any()


def test_find_missed_count_and_indices():
    # tests/test_find_miss.cpp:222-285: missed_size == n - size().
    rng = np.random.default_rng(3)
    t = O.Oracle(1 << 14, dim=8, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 4096)
    t.insert_or_assign(ks, values_for(ks, 8), np.arange(4096, dtype=np.uint64))
    q = np.concatenate([ks[:1000], uniform_keys(rng, 1000, exclude=ks)])
    rng.shuffle(q)
    vals, mk, mi, _ = t.find_missed(q)
    assert mk.size == q.size - 1000
    np.testing.assert_array_equal(q[mi], mk)
    assert np.all(np.diff(mi) > 0)


def test_erase_then_reinsert():
    # tests/test_erase.cpp:29-150
    rng = np.random.default_rng(4)
    t = O.Oracle(1 << 14, dim=8, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 4096)
    vs = values_for(ks, 8)
    t.insert_or_assign(ks, vs, np.arange(4096, dtype=np.uint64))
    t.erase(ks[:1000])
    assert t.size() == 3096
    t.erase(ks[:1000])  # idempotent
    assert t.size() == 3096
    _, f, _ = t.find(ks)
    assert not f[:1000].any() and f[1000:].all()
    t.insert_or_assign(ks[:1000], vs[:1000], np.arange(1000, dtype=np.uint64))
    assert t.size() == 4096
    got, f, _ = t.find(ks)
    assert f.all()
    np.testing.assert_array_equal(got, vs)


@pytest.mark.parametrize("fill", [0.4, 1.0])
def test_reserve_doubles_and_keeps_keys(fill):
    # tests/test_reserve.cpp:173-320: capacity doubles exactly, the size is
    # kept and every key is found with its row, also from load factor 1.0
    # (which exercises the backward-shift defragmentation).
    rng = np.random.default_rng(6)
    n = int((1 << 12) * fill * 1.4)
    ks = uniform_keys(rng, n)
    vs = values_for(ks, 8)
    sc = rng.integers(1, 1 << 40, n, dtype=np.uint64)
    t2 = O.Oracle(1 << 12, 1 << 12, dim=8, strategy=O.CUSTOMIZED)
    t2.insert_or_assign(ks, vs, sc)
    keep, vals0, sc0 = t2.export_batch(1 << 12)
    t = O.Oracle(1 << 12, 1 << 15, dim=8, strategy=O.CUSTOMIZED,
                 max_load_factor=1.0)
    t.insert_or_assign(keep, vals0, sc0)
    assert t.capacity() == 1 << 12
    size0 = t.size()
    assert size0 == keep.size
    if fill == 1.0:
        assert size0 == 1 << 12
    t.reserve(1 << 14)
    assert t.capacity() == 1 << 14
    assert t.size() == size0
    got, f, s = t.find(keep, with_scores=True)
    assert f.all()
    np.testing.assert_array_equal(got, vals0)
    np.testing.assert_array_equal(s, sc0)
    _check_invariants(t)
    t.reserve(1 << 20)  # above max_capacity: the reference leaves it alone
    assert t.capacity() == 1 << 14
    t.reserve(1 << 15)
    assert t.capacity() == 1 << 15
    _check_invariants(t)


def test_auto_growth_on_insert():
    # include/hkv_hashtable.h:1103-1106 with fast_load_factor :3229-3268.
    rng = np.random.default_rng(11)
    t = O.Oracle(1 << 12, 1 << 16, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 5000)
    t.insert_or_assign(ks, values_for(ks, 4), np.arange(5000, dtype=np.uint64))
    assert t.capacity() == 1 << 14  # 5000/4096 > .5, 5000/8192 > .5
    assert t.size() == 5000
    _check_invariants(t)


def test_growth_from_general_capacity():
    # include/table.h:299-311: init = max = 100,000 gives ceil(100000 / 128) =
    # 782 buckets; set_max_capacity (include/hkv_hashtable.h:2955-2977) then
    # lets auto-growth double it once (2 * 200,192 > 2^18).  h mod 2C is
    # h mod C or h mod C + C, so every key stays or moves to bucket b + 782.
    rng = np.random.default_rng(12)
    t = O.Oracle(100_000, 100_000, dim=4, strategy=O.CUSTOMIZED)
    assert t.capacity() == 782 * 128 and t.bucket_count() == 782
    ks = uniform_keys(rng, 40_000)
    t.insert_or_assign(ks, values_for(ks, 4), np.arange(ks.size, dtype=np.uint64))
    t.set_max_capacity(1 << 18)
    more = uniform_keys(rng, 60_000, exclude=ks)
    t.insert_or_assign(more, values_for(more, 4), np.arange(more.size, dtype=np.uint64))
    assert t.capacity() == 1564 * 128
    allk = np.concatenate([ks, more])
    got, f, _ = t.find(allk)
    assert f.all() and t.size() == allk.size
    np.testing.assert_array_equal(got, values_for(allk, 4))
    d, k, s, bsz, v = t.raw()
    live = (k & np.uint64(0xFFFFFFFFFFFFFFFC)) != np.uint64(0xFFFFFFFFFFFFFFFC)
    slot = np.flatnonzero(live).astype(np.uint64)
    home = (murmur3_np(k[live]) % np.uint64(1564 * 128)) // np.uint64(128)
    np.testing.assert_array_equal(slot // np.uint64(128), home)
    _check_invariants(t)


def _check_invariants(t):
    d, k, s, bsz, v = t.raw()
    B = 128
    nb = t.bucket_count()
    live = (k & np.uint64(0xFFFFFFFFFFFFFFFC)) != np.uint64(0xFFFFFFFFFFFFFFFC)
    np.testing.assert_array_equal(bsz, live.reshape(nb, B).sum(1))
    lk = k[live]
    h = murmur3_np(lk)
    np.testing.assert_array_equal(d[live], ((h >> np.uint64(32)) & np.uint64(0xFF)).astype(np.uint8))
    if lk.size:
        _, f, _ = t.find(lk)
        assert f.all()
        assert np.unique(lk).size == lk.size


def test_threaded_mode_matches_single_thread():
    rng = np.random.default_rng(7)
    cap = 1 << 16
    ts = [O.Oracle(cap, dim=4, strategy=O.CUSTOMIZED, threads=th) for th in (1, 4)]
    for rnd in range(6):
        ks = uniform_keys(rng, 20000)
        if rnd:
            ks[:5000] = prev[:5000]
        sc = rng.integers(0, 1 << 20, ks.size, dtype=np.uint64)
        vs = rng.standard_normal((ks.size, 4)).astype(np.float32)
        for t in ts:
            t.insert_or_assign(ks, vs, sc)
        prev = ks
    r0, r1 = ts[0].raw(), ts[1].raw()
    for a, b in zip(r0, r1):
        np.testing.assert_array_equal(a, b)
    _check_invariants(ts[0])
    q = np.concatenate([prev, uniform_keys(rng, 7000)])
    f0, f1 = (t.find(q, np.full((q.size, 4), 9, np.float32), with_scores=True) for t in ts)
    for a, b in zip(f0, f1):
        np.testing.assert_array_equal(a, b)


def test_digest_and_tile_paths_place_identically_without_eviction():
    rng = np.random.default_rng(8)
    a = O.Oracle(1 << 14, dim=4, strategy=O.CUSTOMIZED)
    b = O.Oracle(1 << 14, dim=4, strategy=O.CUSTOMIZED)
    for _ in range(3):
        ks = uniform_keys(rng, 3000)
        sc = rng.integers(0, 1 << 30, 3000, dtype=np.uint64)
        vs = rng.standard_normal((3000, 4)).astype(np.float32)
        a.insert_or_assign(ks, vs, sc, unique_key=True)
        b.insert_or_assign(ks, vs, sc, unique_key=False)
    for x, y in zip(a.raw(), b.raw()):
        np.testing.assert_array_equal(x, y)


def test_sequential_duplicates_last_writer_wins():
    t = O.Oracle(1 << 12, dim=2, strategy=O.CUSTOMIZED)
    ks = np.array([5, 9, 5, 5, 9], np.uint64)
    vs = np.arange(10, dtype=np.float32).reshape(5, 2)
    sc = np.array([1, 2, 3, 4, 5], np.uint64)
    t.insert_or_assign(ks, vs, sc, unique_key=False)
    got, f, s = t.find(np.array([5, 9], np.uint64), with_scores=True)
    assert f.all()
    np.testing.assert_array_equal(got, vs[[3, 4]])
    np.testing.assert_array_equal(s, [4, 5])
    assert t.size() == 2


def test_reserved_keys_are_noops():
    t = O.Oracle(1 << 12, dim=2, strategy=O.CUSTOMIZED)
    ks = np.array([0xFFFFFFFFFFFFFFFF, 0xFFFFFFFFFFFFFFFE, 0xFFFFFFFFFFFFFFFD,
                   0xFFFFFFFFFFFFFFFC, 7], np.uint64)
    t.insert_or_assign(ks, np.ones((5, 2), np.float32), np.ones(5, np.uint64))
    assert t.size() == 1
    _, f, _ = t.find(ks)
    np.testing.assert_array_equal(f, [0, 0, 0, 0, 1])


def test_digest16_tie_break_matches_rank_formula():
    """The lane tournament equals argmin of (score, rank16) with
    rank16(p) = bitrev4((p & 15) ^ (i & 15)) * 8 + (p >> 4)."""
    rng = np.random.default_rng(9)
    cap = 128
    for trial in range(40):
        t = O.Oracle(cap, dim=1, strategy=O.CUSTOMIZED)
        ks = keys_in_bucket(rng, 128, cap, 0)
        sc = rng.integers(0, 3, 128, dtype=np.uint64) + np.uint64(10)
        t.insert_or_assign(ks, np.zeros((128, 1), np.float32), sc)
        d, k0, s0, _, _ = t.raw()
        newk = uniform_keys(rng, 1, exclude=ks)
        idx = int(rng.integers(0, 64))
        batch = np.concatenate([np.full(idx, 0xFFFFFFFFFFFFFFFF, np.uint64), newk])
        t.insert_or_assign(batch, np.zeros((idx + 1, 1), np.float32),
                           np.full(idx + 1, 20, np.uint64))
        _, k1, _, _, _ = t.raw()
        changed = np.nonzero(k0 != k1)[0]
        assert changed.size == 1

        def bitrev4(x):
            return int("{:04b}".format(x)[::-1], 2)
        best = min(range(128), key=lambda p: (int(s0[p]),
                                              bitrev4((p & 15) ^ (idx & 15)) * 8 + (p >> 4)))
        assert changed[0] == best


def test_tile32_tie_break_matches_rank_formula():
    """find_and_lock victim = argmin of (score, rank32) with r = (p - start)
    mod 128 and rank32 = (r & 31) * 4 + (r >> 5)."""
    rng = np.random.default_rng(10)
    cap = 128
    for trial in range(40):
        t = O.Oracle(cap, dim=1, strategy=O.CUSTOMIZED)
        ks = keys_in_bucket(rng, 128, cap, 0)
        sc = rng.integers(0, 3, 128, dtype=np.uint64) + np.uint64(10)
        t.insert_or_assign(ks, np.zeros((128, 1), np.float32), sc)
        _, k0, s0, _, _ = t.raw()
        newk = uniform_keys(rng, 1, exclude=ks)
        start = int(murmur3_np(newk)[0] & np.uint64(127))
        t.insert_or_assign(newk, np.zeros((1, 1), np.float32),
                           np.array([20], np.uint64), unique_key=False)
        _, k1, _, _, _ = t.raw()
        changed = np.nonzero(k0 != k1)[0]
        assert changed.size == 1

        def rank(p):
            r = (p - start) % 128
            return (r & 31) * 4 + (r >> 5)
        best = min(range(128), key=lambda p: (int(s0[p]), rank(p)))
        assert changed[0] == best
