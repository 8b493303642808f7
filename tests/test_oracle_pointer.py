"""Pins the oracle's pointer APIs (find*, find_and_update, find_or_insert*,
lock_keys, unlock_keys) before the GPU is compared with it.

The pointer forms return slot indices here (the GPU returns the addresses of
those slots).  They are pinned by:
  * equality with the already-pinned value APIs where the reference's
    kernels coincide (find_or_insert without locks places keys exactly as the
    value find_or_insert does);
  * the reference's own known-answer tests
    (tests/community/find_or_insert_ptr_lock_test.cpp:1234-1365,
    tests/test_lock_unlock_keys.cpp:96-448);
  * closed forms of the score functors (Lfu sums, Customized assigns);
  * hand-built cases where holding a slot LOCKED changes the outcome.
"""
import numpy as np
import pytest

import oracle as O
from helpers import keys_in_bucket, uniform_keys, values_for

NO = O.NO_SLOT


def _raw_equal(a, b):
    for x, y in zip(a.raw(), b.raw()):
        np.testing.assert_array_equal(x, y)


def _one_bucket_table(strategy, scores_from=1000):
    """128 keys in bucket 0 of a 1024-slot table with scores 1000 + i."""
    rng = np.random.default_rng(5)
    t = O.Oracle(1024, dim=4, strategy=strategy)
    ks = keys_in_bucket(rng, 128, 1024, 0, lo=0, hi=0x3FFFFFFFFFFFFFFF)
    sc = np.arange(scores_from, scores_from + 128, dtype=np.uint64)
    t.insert_or_assign(ks, values_for(ks, 4), sc)
    return t, ks, sc


@pytest.mark.parametrize("strategy", [O.CUSTOMIZED, O.LFU, O.LRU])
def test_ptr_without_locks_places_like_value_find_or_insert(strategy):
    # The non-unique pointer kernel (find_or_insert_ptr_kernel_v2.h:305-386)
    # and the non-unique value kernel both run find_and_lock per key and
    # unlock the key right after it, so the table must come out identical.
    rng = np.random.default_rng(11)
    a = O.Oracle(4096, dim=4, strategy=strategy)
    b = O.Oracle(4096, dim=4, strategy=strategy)
    for r in range(4):
        ks = uniform_keys(rng, 3000)
        ks[::7] = ks[::5][: ks[::7].size]  # repeated keys
        sc = None if strategy == O.LRU else rng.integers(
            1, 1 << 40, size=ks.size, dtype=np.uint64)
        clk = 1000 + r
        a.find_or_insert(ks, np.zeros((ks.size, 4), np.float32), sc,
                         unique_key=False, clock=clk)
        slots, founds = b.find_or_insert_ptr(ks, sc, unique_key=False, clock=clk)
        _raw_equal(a, b)
        # a found key has a slot; the last occurrence of each present key
        # points at the slot that holds it
        assert np.all(founds <= (slots != NO))
        _, keys, _, _, _ = b.raw()
        last = {int(k): i for i, k in enumerate(ks)}
        _, present, _ = b.find(ks)
        for k, i in last.items():
            if present[i]:
                assert slots[i] != NO and keys[int(slots[i])] == k


def test_ptr_unique_without_conflicts_places_like_value_version():
    # No bucket of the batch needs an eviction: the LOCKED hold changes
    # nothing and the layout equals the value find_or_insert's.
    rng = np.random.default_rng(3)
    a = O.Oracle(1 << 14, dim=4, strategy=O.CUSTOMIZED)
    b = O.Oracle(1 << 14, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 4000)
    sc = rng.integers(1, 1 << 40, size=ks.size, dtype=np.uint64)
    a.find_or_insert(ks, np.zeros((ks.size, 4), np.float32), sc)
    slots, founds = b.find_or_insert_ptr(ks, sc)
    _raw_equal(a, b)
    assert not founds.any()
    _, keys, _, _, _ = b.raw()
    np.testing.assert_array_equal(keys[slots.astype(np.int64)], ks)
    # second pass: every key found at the same slot
    s2, f2 = b.find_or_insert_ptr(ks, sc)
    assert f2.all()
    np.testing.assert_array_equal(s2, slots)


def test_lock_hold_keeps_batch_keys_from_eviction():
    # Bucket full with scores 1000..1127.  Key A (score 1000) evicts the
    # score-1000 key; key B (score 1000) then finds A's slot at the minimum.
    # Value find_or_insert: B evicts A.  Pointer find_or_insert with unique
    # keys: A's slot is LOCKED until the batch ends, the minimum over the
    # other slots is 1001 > 1000 and B is refused.
    rng = np.random.default_rng(9)
    t, base, _ = _one_bucket_table(O.CUSTOMIZED)
    new = keys_in_bucket(rng, 2, 1024, 0, lo=0x4000000000000000,
                         hi=0x7FFFFFFFFFFFFFFF)
    sc = np.array([1000, 1000], np.uint64)
    t2, _, _ = _one_bucket_table(O.CUSTOMIZED)
    t2.find_or_insert(new, np.zeros((2, 4), np.float32), sc)
    _, f_val, _ = t2.find(new)
    assert list(f_val) == [False, True]
    slots, founds = t.find_or_insert_ptr(new, sc)
    assert not founds.any()
    assert slots[0] != NO and slots[1] == NO
    _, f_ptr, _ = t.find(new)
    assert list(f_ptr) == [True, False]
    _, keys, scores, _, _ = t.raw()
    assert keys[int(slots[0])] == new[0] and scores[int(slots[0])] == 1000


def test_reference_customized_advanced_kat():
    # tests/community/find_or_insert_ptr_lock_test.cpp:1234-1365: four new
    # keys with scores below the bucket minimum are refused, four present
    # keys take their new scores; the keys are locked and then unlocked.
    rng = np.random.default_rng(21)
    t, base, _ = _one_bucket_table(O.CUSTOMIZED)
    test = keys_in_bucket(rng, 8, 1024, 0, lo=0x3FFFFFFFFFFFFFFF,
                          hi=0xFFFFFFFFFFFFFFFD)
    test[4:8] = base[72:76]
    sc = np.array([20, 78, 97, 98, 99, 1010, 1020, 1035], np.uint64)
    slots, founds = t.find_or_insert_ptr(test, sc, keep_locked=True)
    assert list(founds) == [False] * 4 + [True] * 4
    assert np.all(slots[:4] == NO) and np.all(slots[4:] != NO)
    _, keys, _, _, _ = t.raw()
    assert np.all(keys[slots[4:].astype(np.int64)] == 0xFFFFFFFFFFFFFFFD)
    ok = t.unlock_keys(slots[4:], test[4:])
    assert ok.all()
    assert t.size() == 128
    k, _, s = t.export_batch(1024)
    d = dict(zip(k.tolist(), s.tolist()))
    for i in range(4):
        assert int(test[i]) not in d
    for i in range(4, 8):
        assert d[int(test[i])] == int(sc[i])


@pytest.mark.parametrize("strategy", [O.LFU, O.CUSTOMIZED, O.LRU])
def test_find_ptr_and_find_and_update(strategy):
    rng = np.random.default_rng(4)
    t = O.Oracle(1 << 12, dim=4, strategy=strategy)
    ks = uniform_keys(rng, 1500)
    sc = None if strategy == O.LRU else rng.integers(
        1, 1 << 40, size=ks.size, dtype=np.uint64)
    t.insert_or_assign(ks, values_for(ks, 4), sc, clock=50)
    q = np.concatenate([ks[:700], uniform_keys(rng, 300, exclude=ks),
                        np.array([0xFFFFFFFFFFFFFFFF, 0xFFFFFFFFFFFFFFFC],
                                 np.uint64)])
    slots, founds, s_find = t.find_ptr(q, with_scores=True)
    _, f_val, s_val = t.find(q, with_scores=True)
    np.testing.assert_array_equal(founds, f_val)
    np.testing.assert_array_equal(s_find[founds], s_val[founds])
    _, keys, _, _, _ = t.raw()
    np.testing.assert_array_equal(keys[slots[founds].astype(np.int64)], q[founds])
    assert np.all(slots[~founds] == NO)
    # find_and_update: closed forms of the hit functor
    inp = None if strategy == O.LRU else rng.integers(
        1, 1 << 30, size=q.size, dtype=np.uint64)
    s2, f2, out = t.find_and_update(q, inp, clock=777)
    np.testing.assert_array_equal(s2, slots)
    np.testing.assert_array_equal(f2, founds)
    _, _, after = t.find(q, with_scores=True)
    if strategy == O.LFU:
        np.testing.assert_array_equal(after[founds], s_val[founds] + inp[founds])
    elif strategy == O.CUSTOMIZED:
        np.testing.assert_array_equal(after[founds], inp[founds])
    else:
        assert np.all(after[founds] == 777)
    if inp is not None:
        np.testing.assert_array_equal(out[founds], after[founds])
        np.testing.assert_array_equal(out[~founds], inp[~founds])
    with pytest.raises(O.OracleError) as e:
        t.find_and_update(q, inp, unique_key=False)
    assert e.value.code == 2


def test_lock_unlock_reference_kats():
    # tests/test_lock_unlock_keys.cpp:96-448: existing keys lock and unlock,
    # absent keys fail with null pointers, a partly present batch splits.
    rng = np.random.default_rng(8)
    t = O.Oracle(1 << 12, dim=4, strategy=O.LFU)
    ks = uniform_keys(rng, 1000)
    sc = rng.integers(1, 1 << 30, size=ks.size, dtype=np.uint64)
    t.insert_or_assign(ks, values_for(ks, 4), sc)
    absent = uniform_keys(rng, 200, exclude=ks)
    q = np.concatenate([ks[:300], absent])
    inc = np.full(q.size, 5, np.uint64)
    slots, ok = t.lock_keys(q, inc)
    assert ok[:300].all() and not ok[300:].any()
    assert np.all(slots[300:] == NO)
    _, keys, scores, _, _ = t.raw()
    assert np.all(keys[slots[:300].astype(np.int64)] == 0xFFFFFFFFFFFFFFFD)
    np.testing.assert_array_equal(scores[slots[:300].astype(np.int64)], sc[:300] + 5)
    _, f, _ = t.find(ks[:400])
    assert not f[:300].any() and f[300:].all()
    # a repeated key locks once
    s_rep, ok_rep = t.lock_keys(np.array([ks[500], ks[500]], np.uint64), inc[:2])
    assert list(ok_rep) == [True, False]
    ok_un = t.unlock_keys(np.concatenate([slots, s_rep]),
                          np.concatenate([q, [ks[500], ks[500]]]).astype(np.uint64))
    assert ok_un[:300].all() and not ok_un[300:500].any()
    assert list(ok_un[500:]) == [True, False]
    _, f, _ = t.find(ks)
    assert f.all()


def test_locked_victim_is_refused():
    # Every key of the full bucket is LOCKED: no slot is eligible, the start
    # slot holds LOCKED, and an insert is refused instead of taking it.
    rng = np.random.default_rng(12)
    t, base, _ = _one_bucket_table(O.CUSTOMIZED)
    slots, ok = t.lock_keys(base, np.full(128, 5000, np.uint64))
    assert ok.all()
    new = keys_in_bucket(rng, 3, 1024, 0, lo=0x4000000000000000,
                         hi=0x7FFFFFFFFFFFFFFF)
    t.insert_or_assign(new, values_for(new, 4), np.full(3, 1 << 60, np.uint64))
    _, f, _ = t.find(new)
    assert not f.any()
    assert t.unlock_keys(slots, base).all()
    t.insert_or_assign(new, values_for(new, 4), np.full(3, 1 << 60, np.uint64))
    _, f, _ = t.find(new)
    assert f.all()


def test_keep_locked_requires_unique_keys():
    t = O.Oracle(1024, dim=4, strategy=O.CUSTOMIZED)
    with pytest.raises(O.OracleError) as e:
        t.find_or_insert_ptr(np.arange(4, dtype=np.uint64),
                             np.ones(4, np.uint64), unique_key=False,
                             keep_locked=True)
    assert e.value.code == 3


@pytest.mark.parametrize("strategy", [O.LFU, O.CUSTOMIZED, O.LRU, O.EPOCH_LFU])
def test_assign_contains_closed_forms(strategy):
    # contains = find's founds; assign = assign_scores (pinned separately)
    # plus the input row on present keys; assign_values = the row only.
    rng = np.random.default_rng(31)
    mk = lambda: O.Oracle(1 << 12, dim=4, strategy=strategy)
    a, b, c = mk(), mk(), mk()
    for t in (a, b, c):
        t.set_global_epoch(2)
    ks = uniform_keys(rng, 1500)
    sc = None if strategy == O.LRU else rng.integers(1, 1 << 30, size=ks.size,
                                                      dtype=np.uint64)
    for t in (a, b, c):
        t.insert_or_assign(ks, values_for(ks, 4), sc, clock=10)
    q = np.concatenate([ks[:800], uniform_keys(rng, 400, exclude=ks),
                        np.array([0xFFFFFFFFFFFFFFFF], np.uint64)])
    _, f, _ = a.find(q)
    np.testing.assert_array_equal(a.contains(q), f)
    inp = None if strategy == O.LRU else rng.integers(1, 1 << 30, size=q.size,
                                                      dtype=np.uint64)
    rows = rng.standard_normal((q.size, 4)).astype(np.float32)
    a.assign(q, rows, inp, clock=99)
    b.assign_scores(q, inp, clock=99)
    c.assign_values(q, rows)
    _, ka, sa, ba, va = a.raw()
    _, kb, sb, bb, vb = b.raw()
    _, kc, scc, bc, vc = c.raw()
    np.testing.assert_array_equal(ka, kb)
    np.testing.assert_array_equal(sa, sb)
    np.testing.assert_array_equal(ba, bb)
    np.testing.assert_array_equal(va, vc)
    got, found, _ = a.find(q)
    np.testing.assert_array_equal(got[found], rows[found])
    assert a.size() == 1500
    # assign_values leaves scores as inserted
    x = O.Oracle(1 << 12, dim=4, strategy=strategy)
    x.set_global_epoch(2)
    x.insert_or_assign(ks, values_for(ks, 4), sc, clock=10)
    np.testing.assert_array_equal(scc, x.raw()[2])


def _np_pred(kind, k, s, pat, th):
    if kind == 0:
        return s < np.uint64(th)
    if kind == 1:
        return s >= np.uint64(th)
    if kind == 2:
        return s > np.uint64(th)
    if kind == 3:
        return (k & np.uint64(pat)) == np.uint64(pat)
    return ((k & np.uint64(0x7F)) > np.uint64(pat)) & (s > np.uint64(th))


@pytest.mark.parametrize("kind,pat,th", [(0, 0, 500), (1, 0, 500), (2, 0, 900),
                                         (3, 0x5, 0), (4, 0x3F, 300)])
def test_predicate_apis_closed_forms(kind, pat, th):
    # size_if / export_batch_if / erase_if against the same predicate
    # evaluated by numpy over the full export (include/hkv_hashtable.h:
    # 2409-2441, 2623-2672, 2829-2845).
    rng = np.random.default_rng(40 + kind)
    t = O.Oracle(1 << 13, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 3000)
    sc = rng.integers(0, 1000, size=ks.size, dtype=np.uint64)
    t.insert_or_assign(ks, values_for(ks, 4), sc)
    k, v, s = t.export_batch(1 << 13)
    m = _np_pred(kind, k, s, pat, th)
    assert t.size_if(kind, pat, th) == int(m.sum())
    ek, ev, es = t.export_batch_if(kind, pat, th, 1 << 13)
    np.testing.assert_array_equal(ek, k[m])
    np.testing.assert_array_equal(es, s[m])
    np.testing.assert_array_equal(ev, v[m])
    # a window [offset, offset + n) of slots
    wk, _, _ = t.export_batch_if(kind, pat, th, 2000, offset=3000)
    k2, _, s2 = t.export_batch(2000, 3000)
    np.testing.assert_array_equal(wk, k2[_np_pred(kind, k2, s2, pat, th)])
    assert t.erase_if(kind, pat, th) == int(m.sum())
    assert t.size() == 3000 - int(m.sum())
    _, f, _ = t.find(k)
    np.testing.assert_array_equal(f, ~m)
    assert t.size_if(kind, pat, th) == 0


def test_set_max_capacity_unblocks_growth():
    t = O.Oracle(1024, 1024, dim=4, strategy=O.CUSTOMIZED)
    rng = np.random.default_rng(2)
    with pytest.raises(O.OracleError) as e:
        t.set_max_capacity(3000)
    assert e.value.code == 3
    ks = uniform_keys(rng, 900)
    t.insert_or_assign(ks, values_for(ks, 4), np.ones(900, np.uint64))
    assert t.capacity() == 1024
    t.set_max_capacity(4096)
    ks2 = uniform_keys(rng, 900, exclude=ks)
    t.insert_or_assign(ks2, values_for(ks2, 4), np.ones(900, np.uint64))
    assert t.capacity() == 4096
