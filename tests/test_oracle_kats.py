"""Pins the oracle's find_or_insert, accum_or_assign and assign_scores to the
known answers of the reference's own tests.

* find_or_insert: tests/test_find_or_insert.cpp:707-842 (a second call on
  present keys returns the stored rows, not the new inputs; a mixed batch
  adds only its new keys) and
  tests/test_find_or_insert_evict_strategies.cpp:560-640 (scores after two
  calls: Lru later clock, Lfu 2x, EpochLru epoch 123 and a later clock,
  EpochLfu epoch 123 and 2x frequency, Customized the input).
* accum_or_assign: tests/test_accum_or_assign.cpp:196-420 (Lru),
  :423-640 (Lfu) and :860-1045 (EpochLfu with a saturating frequency):
  table size by flag, accumulated row == key * 0.00002, rows and scores of
  flag-mismatched keys unchanged.
* assign_scores: tests/test_assign_scores.cpp:101-375, 681-760, 1110-1260
  (present keys' scores change, absent keys are ignored, the size is kept,
  repeated keys with unique_key=false).  The reference asserts only that
  scores change; the exact values asserted here are the
  update_without_missed closed forms (Lfu old + in, EpochLfu epoch | sat.
  sum, Customized in, Lru clock), whose arithmetic the score-functor known
  answers of tests/test_score_functor/test_score_functor.cpp:162-473 pin.

Each check fails for a plausible slip: rows copied in instead of out, the
new input stored over a present row, a score rule applied on the wrong
path, a flag test inverted, an absent key inserted by assign_scores.

Every test runs on the oracle (CPU) and, under the gpu marker, unchanged on
the gfx950 table through the C ABI, so these known answers hold for both.
"""
import numpy as np
import pytest

import oracle as O
from helpers import keys_in_bucket, values_for

U32 = 0xFFFFFFFF


@pytest.fixture(params=["oracle", pytest.param("gfx950", marks=pytest.mark.gpu)])
def make(request):
    if request.param == "oracle":
        return O.Oracle
    from gpu_pair import GpuTable
    return GpuTable


def continuous(n, start=1, dim=8):
    """create_continuous_keys (tests/common/test_util.h:213-242): keys
    start..start+n-1, scores equal to the keys, rows key * 0.00001."""
    k = np.arange(start, start + n, dtype=np.uint64)
    return k, k.copy(), values_for(k, dim)


def epochlfu_expected(epoch, score):
    """make_expected_score_for_epochlfu (tests/common/test_util.h:319-324)."""
    lo = U32 if score >= U32 else score & U32
    return (epoch << 32) | lo


# -- find_or_insert -----------------------------------------------------------

def test_find_or_insert_returns_stored_rows_on_second_call(make):
    # tests/test_find_or_insert.cpp:707-842 (kLru, 128K slots, dim 8).
    cap, dim, n = 128 * 1024, 8, 1024
    t = make(cap, dim=dim, strategy=O.LRU)
    k, _, v = continuous(n, dim=dim)
    out = t.find_or_insert(k, v.copy(), clock=100)
    assert t.size() == n
    np.testing.assert_array_equal(out, v)  # new keys keep (and insert) the input
    new_v = np.repeat((np.arange(n) * 0.00002).astype(np.float32)[:, None], dim, 1)
    out2 = t.find_or_insert(k, new_v.copy(), clock=200)
    assert t.size() == n
    np.testing.assert_array_equal(out2, v)  # stored rows come out, inputs ignored
    # mixed: the 1024 old keys plus 1024 new ones (i + 10001), rows i + 201
    mk = np.concatenate([np.arange(1, 1025), np.arange(1024, 2048) + 10001]).astype(np.uint64)
    mv = np.repeat((np.arange(2048) + 201).astype(np.float32)[:, None], dim, 1)
    out3 = t.find_or_insert(mk, mv.copy(), clock=300)
    assert t.size() == n + 1024
    np.testing.assert_array_equal(out3[:1024], v)
    np.testing.assert_array_equal(out3[1024:], mv[1024:])
    got, f, _ = t.find(mk)
    assert f.all()
    np.testing.assert_array_equal(got[1024:], mv[1024:])
    np.testing.assert_array_equal(got[:1024], v)


@pytest.mark.parametrize("unique", [True, False])
@pytest.mark.parametrize("strategy", [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU,
                                      O.CUSTOMIZED])
def test_find_or_insert_scores_by_strategy(make, strategy, unique):
    # tests/test_find_or_insert_evict_strategies.cpp:405-640.
    cap, dim, n, epoch = 128 * 1024, 8, 1024, 123
    t = make(cap, dim=dim, strategy=strategy)
    if strategy in (O.EPOCH_LRU, O.EPOCH_LFU):
        t.set_global_epoch(epoch)
    k, sc, v = continuous(n, dim=dim)
    sp = None if strategy in (O.LRU, O.EPOCH_LRU) else sc
    c1, c2 = 5 << 20, 9 << 20  # two clocks, the second later
    t.find_or_insert(k, v.copy(), sp, unique_key=unique, clock=c1)
    assert t.size() == n
    _, f, first = t.find(k, with_scores=True)
    assert f.all()
    out = t.find_or_insert(k, np.zeros_like(v), sp, unique_key=unique, clock=c2)
    assert t.size() == n
    np.testing.assert_array_equal(out, v)
    _, f, s = t.find(k, with_scores=True)
    assert f.all()
    if strategy == O.LRU:
        assert (s > 0).all() and (s > first).all()
        assert (s == c2).all()
    elif strategy == O.LFU:
        np.testing.assert_array_equal(s, 2 * sc)
    elif strategy == O.EPOCH_LRU:
        assert ((s >> np.uint64(32)) == epoch).all()
        lo = s & np.uint64(U32)
        assert (lo > 0).all() and (lo > (first & np.uint64(U32))).all()
        assert (lo == np.uint64((c2 >> 20) & U32)).all()
    elif strategy == O.EPOCH_LFU:
        assert ((s >> np.uint64(32)) == epoch).all()
        np.testing.assert_array_equal(s & np.uint64(U32), 2 * (sc & np.uint64(U32)))
    else:
        np.testing.assert_array_equal(s, sc)


# -- accum_or_assign ------------------------------------------------------------

def _accum_fixture(rng, freq_range=None):
    """tests/test_accum_or_assign.cpp:196-250: 128 base keys and 4 test keys
    in bucket 1 of an 8-bucket table; base flags random with 72 and 73
    false; test keys 2 and 3 are base keys 72 and 73 with flags true and
    false; rows key * 0.00001."""
    cap, dim = 8 * 128, 16
    base = keys_in_bucket(rng, 128, cap, 1, lo=0, hi=0x3FFFFFFFFFFFFFFF)
    test = keys_in_bucket(rng, 4, cap, 1, lo=0x3FFFFFFFFFFFFFFF,
                          hi=0xFFFFFFFFFFFFFFFD)
    fb = rng.random(128) < 0.5
    ft = rng.random(4) < 0.5
    fb[72] = fb[73] = False
    test[2], test[3] = base[72], base[73]
    ft[2], ft[3] = True, False
    return cap, dim, base, test, fb, ft


@pytest.mark.parametrize("seed", range(4))
def test_accum_or_assign_lru_kat(make, seed):
    # tests/test_accum_or_assign.cpp:196-420 (kLru, no input scores).
    rng = np.random.default_rng(300 + seed)
    cap, dim, base, test, fb, ft = _accum_fixture(rng)
    t = make(cap, dim=dim, strategy=O.LRU)
    c1, c2 = 1000, 2000
    t.accum_or_assign(base, values_for(base, dim), fb.astype(np.uint8), clock=c1)
    assert t.size() == int((~fb).sum())
    k, v, s = t.export_batch(cap)
    assert k.size == int((~fb).sum())
    assert set(k.tolist()) == set(base[~fb].tolist())
    np.testing.assert_array_equal(v, values_for(k, dim))
    assert (s == c1).all()
    t.accum_or_assign(test, values_for(test, dim), ft.astype(np.uint8), clock=c2)
    new = np.array([x not in set(base.tolist()) for x in test])
    assert t.size() == int((~fb).sum()) + int((new & ~ft).sum())
    k, v, s = t.export_batch(cap)
    assert k.size == t.size()
    for key, row, sc in zip(k, v, s):
        if key == test[2]:
            np.testing.assert_array_equal(row, np.float32(int(key) * 0.00002))
            assert sc == c2
        else:
            np.testing.assert_array_equal(row, np.float32(int(key) * 0.00001))
            newk = key in set(test.tolist()) and key != test[3]
            assert sc == (c2 if newk else c1)


@pytest.mark.parametrize("seed", range(4))
def test_accum_or_assign_lfu_kat(make, seed):
    # tests/test_accum_or_assign.cpp:423-640 (kLfu, scores key % 1000).
    rng = np.random.default_rng(310 + seed)
    cap, dim, base, test, fb, ft = _accum_fixture(rng)
    fr = 1000
    t = make(cap, dim=dim, strategy=O.LFU)
    t.accum_or_assign(base, values_for(base, dim), fb.astype(np.uint8), base % np.uint64(fr))
    assert t.size() == int((~fb).sum())
    k, v, s = t.export_batch(cap)
    np.testing.assert_array_equal(s, k % np.uint64(fr))
    np.testing.assert_array_equal(v, values_for(k, dim))
    ts = test % np.uint64(fr)
    t.accum_or_assign(test, values_for(test, dim), ft.astype(np.uint8), ts)
    new = np.array([x not in set(base.tolist()) for x in test])
    assert t.size() == int((~fb).sum()) + int((new & ~ft).sum())
    k, v, s = t.export_batch(cap)
    acc = k == test[2]
    assert acc.sum() == 1
    np.testing.assert_array_equal(s[acc], (k[acc] % np.uint64(fr)) * np.uint64(2))
    np.testing.assert_array_equal(v[acc], values_for(k[acc], dim) * np.float32(2))
    np.testing.assert_array_equal(v[acc][0], np.float32(int(test[2]) * 0.00002))
    np.testing.assert_array_equal(s[~acc], k[~acc] % np.uint64(fr))
    np.testing.assert_array_equal(v[~acc], values_for(k[~acc], dim))


@pytest.mark.parametrize("seed", range(4))
def test_accum_or_assign_epoch_lfu_kat(make, seed):
    # tests/test_accum_or_assign.cpp:860-1045 (kEpochLfu): base key 71 enters
    # with frequency 2^32 - 2, and accumulating it again saturates the low
    # word; untouched base keys keep epoch 1, touched keys get epoch 2.
    rng = np.random.default_rng(320 + seed)
    cap, dim, base, test, fb, ft = _accum_fixture(rng)
    fr = 1000
    fb[71] = False
    sb = base % np.uint64(fr)
    sb[71] = np.uint64(U32 - 1)
    test[1] = base[71]
    ft[1] = True
    ts = test % np.uint64(fr)
    ts[1] = sb[71]
    t = make(cap, dim=dim, strategy=O.EPOCH_LFU)
    t.set_global_epoch(1)
    t.accum_or_assign(base, values_for(base, dim), fb.astype(np.uint8), sb)
    assert t.size() == int((~fb).sum())
    k, v, s = t.export_batch(cap)
    for key, sc in zip(k, s):
        want = int(sb[71]) if key == base[71] else int(key) % fr
        assert int(sc) == epochlfu_expected(1, want)
    np.testing.assert_array_equal(v, values_for(k, dim))
    t.set_global_epoch(2)
    t.accum_or_assign(test, values_for(test, dim), ft.astype(np.uint8), ts)
    bs = set(base.tolist())
    new = np.array([x not in bs for x in test])
    assert t.size() == int((~fb).sum()) + int((new & ~ft).sum())
    k, v, s = t.export_batch(cap)
    assert base[71] in set(k.tolist())
    for key, row, sc in zip(k, v, s):
        key = int(key)
        if key in (int(test[1]), int(test[2])):
            want = int(sb[71]) * 2 if key == int(base[71]) else (key % fr) * 2
            assert int(sc) == epochlfu_expected(2, want)
            np.testing.assert_array_equal(row, np.float32(key * 0.00002))
        else:
            assert int(sc) == epochlfu_expected(2 - int(key in bs), key % fr)
            np.testing.assert_array_equal(row, np.float32(key * 0.00001))


# -- assign_scores --------------------------------------------------------------

def test_assign_scores_basic_and_partial(make):
    # tests/test_assign_scores.cpp:101-178 (basic_function) and :301-375
    # (partial_keys_exist), kLfu, dim 8.
    cap, dim = 128 * 1024, 8
    t = make(cap, dim=dim, strategy=O.LFU)
    k, sc, v = continuous(1024, dim=dim)
    t.insert_or_assign(k, v, sc)
    t.assign_scores(k, sc + np.uint64(1000))
    _, f, s = t.find(k, with_scores=True)
    assert f.all() and (s != sc).all()
    np.testing.assert_array_equal(s, 2 * sc + np.uint64(1000))  # old + in

    t = make(cap, dim=dim, strategy=O.LFU)
    k, sc, v = continuous(500, dim=dim)
    t.insert_or_assign(k, v, sc)
    uk = np.arange(1, 1001, dtype=np.uint64)
    t.assign_scores(uk, np.uint64(5000) + np.arange(1000, dtype=np.uint64))
    assert t.size() == 500  # absent keys ignored
    _, f, s = t.find(k, with_scores=True)
    assert f.all() and (s != sc).all()
    np.testing.assert_array_equal(s, sc + np.uint64(5000) + np.arange(500, dtype=np.uint64))
    _, f2, _ = t.find(uk[500:])
    assert not f2.any()
    got, _, _ = t.find(k)
    np.testing.assert_array_equal(got, v)  # rows untouched


def test_assign_scores_single_key_epoch_lfu_and_empty_table(make):
    # tests/test_assign_scores.cpp:180-214 (empty table) and :236-299
    # (single key, kEpochLfu, epoch 1, score 100 then 99999).
    t = make(128 * 1024, dim=8, strategy=O.LFU)
    k, sc, _ = continuous(100)
    t.assign_scores(k, sc)
    assert t.size() == 0
    t = make(128 * 1024, dim=8, strategy=O.EPOCH_LFU)
    t.set_global_epoch(1)
    key = np.array([12345], np.uint64)
    t.insert_or_assign(key, np.full((1, 8), 1.5, np.float32), np.array([100], np.uint64))
    t.assign_scores(key, np.array([99999], np.uint64))
    _, f, s = t.find(key, with_scores=True)
    assert f[0] and s[0] != 100
    assert int(s[0]) == (1 << 32) | (100 + 99999)


def test_assign_scores_repeated_updates_and_duplicates(make):
    # tests/test_assign_scores.cpp:681-750 (multiple_updates) and
    # :1183-1260 (unique_key=false, each key repeated with one score).
    cap, dim, n = 128 * 1024, 8, 1024
    t = make(cap, dim=dim, strategy=O.LFU)
    k, sc, v = continuous(n, dim=dim)
    t.insert_or_assign(k, v, sc)
    want = sc.copy()
    for r in range(3):
        inc = np.uint64((r + 1) * 1000) + np.arange(n, dtype=np.uint64)
        t.assign_scores(k, inc)
        want = want + inc
        _, f, s = t.find(k, with_scores=True)
        assert f.all()
        np.testing.assert_array_equal(s, want)
    rep, target = 4, 77
    bk = np.repeat(k[:256], rep)
    t.assign_scores(bk, np.full(bk.size, target, np.uint64))
    _, _, s = t.find(k, with_scores=True)
    np.testing.assert_array_equal(s[:256], want[:256] + np.uint64(rep * target))
    np.testing.assert_array_equal(s[256:], want[256:])


@pytest.mark.parametrize("strategy", [O.LRU, O.EPOCH_LRU, O.CUSTOMIZED])
def test_assign_scores_other_strategies(make, strategy):
    # update_without_missed: Lru the call's clock, EpochLru epoch | clock >> 20,
    # Customized the input (include/score_functor.h).
    cap, dim, n = 1 << 14, 4, 512
    t = make(cap, dim=dim, strategy=strategy)
    if strategy == O.EPOCH_LRU:
        t.set_global_epoch(9)
    k, sc, v = continuous(n, dim=dim)
    sp = sc if strategy == O.CUSTOMIZED else None
    t.insert_or_assign(k, v, sp, clock=3 << 20)
    t.assign_scores(k, None if sp is None else sc * np.uint64(3), clock=7 << 20)
    _, f, s = t.find(k, with_scores=True)
    assert f.all()
    if strategy == O.LRU:
        assert (s == (7 << 20)).all()
    elif strategy == O.EPOCH_LRU:
        assert (s == ((9 << 32) | 7)).all()
    else:
        np.testing.assert_array_equal(s, sc * np.uint64(3))
