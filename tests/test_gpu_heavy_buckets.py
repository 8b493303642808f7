"""GPU parity for duplicate-heavy batches: buckets that receive many
occurrences of a few keys in one call.

Each case mixes hot keys (hundreds to thousands of occurrences, some present
in the table before the call, some new) with light keys, and compares the
GPU table with the oracle bit-exactly after every call: full exports, rows
returned by find_or_insert and evicted records.  Buckets whose new keys fit
their EMPTY slots take the folded path; full or nearly full tables take the
serial batch-order walk.
"""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, records_equal
from helpers import keys_in_bucket, uniform_keys

pytestmark = pytest.mark.gpu

STRATS = [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU, O.CUSTOMIZED]


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def hot_batch(rng, present, fresh, reps, light):
    """Hot keys (present and fresh) repeated `reps` times each, plus light
    keys, shuffled."""
    hot = np.concatenate([present, fresh])
    q = np.concatenate([np.repeat(hot, reps), light])
    return q[rng.permutation(q.size)]


def scores_for(strategy, rng, n, big=False):
    if strategy in (O.LRU, O.EPOCH_LRU):
        return None
    if big and strategy == O.LFU:
        return rng.integers(1 << 60, 1 << 63, n, dtype=np.uint64)  # sums wrap
    if big and strategy == O.EPOCH_LFU:
        return rng.integers(1 << 30, 1 << 32, n, dtype=np.uint64)  # saturates
    return rng.integers(0, 1000, n, dtype=np.uint64)




def _run(p, op, rng, q, strategy, dim, clock, big=False, unique=False):
    sc = scores_for(strategy, rng, q.size, big)
    v = rand_vals(rng, q.size, dim)
    if op == "insert_or_assign":
        p.insert_or_assign(q, v, sc, unique_key=unique, clock=clock)
    elif op == "find_or_insert":
        ov, gv = p.find_or_insert(q, v, sc, unique_key=unique, clock=clock)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    elif op == "insert_and_evict":
        o, g = p.insert_and_evict(q, v, sc, unique_key=unique, clock=clock)
        records_equal(o, g)
    else:
        p.assign_scores(q, sc, clock=clock)
    p.assert_same_state()


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert",
                                "insert_and_evict", "assign_scores"])
@pytest.mark.parametrize("strategy", STRATS)
def test_hot_keys_fit(op, strategy):
    """Hot keys whose buckets keep EMPTY slots: the folded path."""
    rng = np.random.default_rng(300 + strategy)
    cap, dim = 1 << 15, 8
    p = Pair(cap, dim=dim, strategy=strategy)
    p.set_global_epoch(4)
    base = uniform_keys(rng, 6000)
    p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                       scores_for(strategy, rng, base.size), clock=10)
    p.assert_same_state()
    for r in range(3):
        p.set_global_epoch(5 + r)
        present = rng.choice(base, 12, replace=False)
        fresh = uniform_keys(rng, 10, exclude=base)
        light = uniform_keys(rng, 900, exclude=np.concatenate([base, fresh]))
        q = hot_batch(rng, present, fresh, rng.integers(40, 700), light)
        _run(p, op, rng, q, strategy, dim, clock=20 + r, big=(r == 2))
        base = np.concatenate([base, fresh])


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert",
                                "insert_and_evict"])
@pytest.mark.parametrize("strategy", STRATS)
def test_hot_keys_full_buckets(op, strategy):
    """Hot keys into buckets without room: the serial walk, with eviction."""
    rng = np.random.default_rng(320 + strategy)
    cap, dim = 1 << 12, 4
    p = Pair(cap, dim=dim, strategy=strategy)
    p.set_global_epoch(2)
    base = uniform_keys(rng, 6000)
    p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                       scores_for(strategy, rng, base.size), clock=10)
    p.assert_same_state()
    (res, _, _), _ = p.export()
    present = rng.choice(res, 6, replace=False)
    fresh = uniform_keys(rng, 8, exclude=base)
    q = hot_batch(rng, present, fresh, 300, uniform_keys(rng, 400, exclude=base))
    _run(p, op, rng, q, strategy, dim, clock=30)


@pytest.mark.parametrize("strategy", [O.LFU, O.EPOCH_LFU, O.CUSTOMIZED])
def test_many_heavy_buckets_in_one_partition(strategy):
    """40 heavy buckets in one 256-bucket partition (more than the block's 16
    groups take in one round), plus enough light keys that the rest of the
    partition needs several runs."""
    rng = np.random.default_rng(340 + strategy)
    cap, dim = 1 << 15, 4   # 256 buckets: a single partition
    p = Pair(cap, dim=dim, strategy=strategy)
    p.set_global_epoch(1)
    base = uniform_keys(rng, 3000)
    p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                       scores_for(strategy, rng, base.size), clock=10)
    # 40 buckets with 6 new hot keys each; 4 of them with 130, more than
    # their EMPTY slots (those take the serial walk)
    hot = [keys_in_bucket(rng, 130 if b < 4 else 6, cap, b * 5 + 1,
                          lo=1 << 40, hi=1 << 62) for b in range(40)]
    (res, _, _), _ = p.export()
    hotk = np.concatenate(hot)
    q = np.concatenate([np.repeat(hotk, 40), rng.choice(res, 2000),
                        uniform_keys(rng, 3000, exclude=np.concatenate([base, hotk]))])
    q = q[rng.permutation(q.size)]
    for op in ("find_or_insert", "insert_or_assign"):
        _run(p, op, rng, q, strategy, dim, clock=40)


def test_exact_fit_of_new_keys():
    """A heavy bucket whose new distinct keys equal its EMPTY slots, then one
    more than fit."""
    rng = np.random.default_rng(360)
    cap, dim = 1 << 14, 4
    p = Pair(cap, dim=dim, strategy=O.CUSTOMIZED)
    b = 7
    ks = keys_in_bucket(rng, 128, cap, b)
    p.insert_or_assign(ks[:100], rand_vals(rng, 100, dim),
                       rng.integers(0, 100, 100, dtype=np.uint64))
    q = np.concatenate([np.repeat(ks[100:128], 20), np.repeat(ks[:5], 30)])
    q = q[rng.permutation(q.size)]
    _run(p, "find_or_insert", rng, q, O.CUSTOMIZED, dim, clock=1)
    more = keys_in_bucket(rng, 140, cap, b)[128:]
    q = np.concatenate([np.repeat(more, 40), np.repeat(ks[:3], 40)])
    q = q[rng.permutation(q.size)]
    _run(p, "insert_or_assign", rng, q, O.CUSTOMIZED, dim, clock=2)


def test_epoch_lfu_ignored_epoch_fold():
    """find_or_insert with ignore_evict_strategy on an EpochLfu table whose
    epoch is unset: desired scores are the inputs themselves."""
    rng = np.random.default_rng(361)
    cap, dim = 1 << 14, 4
    p = Pair(cap, dim=dim, strategy=O.EPOCH_LFU)
    base = uniform_keys(rng, 1000)
    sc = rng.integers(0, 1 << 40, base.size, dtype=np.uint64)
    ov, gv = p.find_or_insert(base, rand_vals(rng, base.size, dim), sc, unique_key=False,
                              ignore=True)
    np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    q = hot_batch(rng, base[:5], uniform_keys(rng, 5, exclude=base), 200,
                  uniform_keys(rng, 300, exclude=base))
    s2 = rng.integers(0, 1 << 40, q.size, dtype=np.uint64)
    ov, gv = p.find_or_insert(q, rand_vals(rng, q.size, dim), s2, unique_key=False,
                              ignore=True)
    np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    p.assert_same_state()


def test_single_key_repeated_many_times():
    """One key 50,000 times (new, then present), as a Zipf head produces."""
    rng = np.random.default_rng(362)
    cap, dim = 1 << 16, 32
    for strategy in (O.EPOCH_LFU, O.LFU, O.LRU):
        p = Pair(cap, dim=dim, strategy=strategy)
        p.set_global_epoch(3)
        k = uniform_keys(rng, 1)
        light = uniform_keys(rng, 2000, exclude=k)
        for r in range(2):
            q = np.concatenate([np.repeat(k, 50000), light])
            q = q[rng.permutation(q.size)]
            _run(p, "find_or_insert", rng, q, strategy, dim, clock=5 + r)


def _long_bucket_batch(rng, p, cap, dim, strategy):
    """Batches whose partitions (256 buckets) hold at most 704 entries but
    some buckets more than 32: k_apply_fast applies the short buckets and
    lists the partition for its long ones only.  Bucket kinds: a few hot keys
    (present and new) repeated; 40 distinct new keys once each; a nearly full
    bucket given 5 new hot keys (no fold: the batch-order walk, with
    eviction); 140 distinct keys (more than a bucket holds)."""
    nb = cap // 128
    parts = rng.choice(nb // 256, 12, replace=False)
    fill, batch = [], []
    for j, part in enumerate(parts):
        b = int(part) * 256 + int(rng.integers(0, 256))
        kind = j % 4
        if kind == 0:
            ks = keys_in_bucket(rng, 4, cap, b, lo=1 << 40, hi=1 << 62)
            fill.append(ks[:2])
            batch.append(np.repeat(ks, rng.integers(10, 41)))
        elif kind == 1:
            batch.append(keys_in_bucket(rng, 40, cap, b, lo=1 << 40, hi=1 << 62))
        elif kind == 2:
            ks = keys_in_bucket(rng, 130, cap, b, lo=1 << 40, hi=1 << 62)
            fill.append(ks[:125])
            batch.append(np.concatenate([np.repeat(ks[125:], 10), np.repeat(ks[:3], 5)]))
        else:
            batch.append(keys_in_bucket(rng, 140, cap, b, lo=1 << 40, hi=1 << 62))
    return np.concatenate(fill), np.concatenate(batch)


@pytest.mark.parametrize("op", ["find_or_insert", "insert_or_assign", "insert_and_evict",
                                "assign_scores"])
@pytest.mark.parametrize("strategy", STRATS)
def test_long_buckets_in_small_partitions(op, strategy):
    rng = np.random.default_rng(380 + strategy)
    cap, dim = 1 << 20, 4
    p = Pair(cap, dim=dim, strategy=strategy)
    p.set_global_epoch(6)
    fill, hot = _long_bucket_batch(rng, p, cap, dim, strategy)
    base = np.concatenate([fill, uniform_keys(rng, 1 << 17, exclude=fill)])
    p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                       scores_for(strategy, rng, base.size), clock=10)
    p.assert_same_state()
    for r in range(2):
        p.set_global_epoch(7 + r)
        light = np.concatenate([rng.choice(base, 1500),
                                uniform_keys(rng, 3000, exclude=np.concatenate([base, hot]))])
        q = np.concatenate([hot, light])
        q = q[rng.permutation(q.size)]
        _run(p, op if r else "find_or_insert", rng, q, strategy, dim, clock=50 + r,
             big=(r == 1))


def test_long_buckets_accum():
    """The same batches through accum_or_assign, which lists whole
    partitions (its accumulations run in batch order, without a fold)."""
    rng = np.random.default_rng(399)
    cap, dim = 1 << 20, 4
    for strategy in (O.LFU, O.CUSTOMIZED):
        p = Pair(cap, dim=dim, strategy=strategy)
        fill, hot = _long_bucket_batch(rng, p, cap, dim, strategy)
        base = np.concatenate([fill, uniform_keys(rng, 1 << 16, exclude=fill)])
        p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                           scores_for(strategy, rng, base.size), clock=10)
        q = np.concatenate([hot, rng.choice(base, 1000), uniform_keys(rng, 2000, exclude=base)])
        q = q[rng.permutation(q.size)]
        flags = (rng.random(q.size) < 0.5).astype(np.uint8)
        p.accum_or_assign(q, rng.uniform(-0.01, 0.01, (q.size, dim)).astype(np.float32), flags,
                          scores_for(strategy, rng, q.size), clock=11)
        p.assert_same_state()


@pytest.mark.parametrize("op", ["find_or_insert", "insert_or_assign", "insert_and_evict",
                                "assign_scores"])
@pytest.mark.parametrize("strategy", STRATS)
def test_partitions_beyond_one_load(op, strategy):
    """Partitions of 705-4096 entries (hot keys repeated hundreds of times)
    go to the multi-run kernel whole: its fold takes the hot buckets and its
    run loop the short ones, including a partition with more short-bucket
    entries than one LDS run holds (36 buckets of 22 keys of their own, in
    partition 3)."""
    rng = np.random.default_rng(420 + strategy)
    cap, dim = 1 << 17, 4
    p = Pair(cap, dim=dim, strategy=strategy)
    p.set_global_epoch(6)
    base = uniform_keys(rng, 40000)
    p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                       scores_for(strategy, rng, base.size), clock=10)
    p.assert_same_state()
    crowd = np.concatenate([keys_in_bucket(rng, 22, cap, 768 + 7 * j, lo=1 << 40, hi=1 << 62)
                            for j in range(36)])
    for r in range(3):
        p.set_global_epoch(7 + r)
        fresh = uniform_keys(rng, 602, exclude=np.concatenate([base, crowd]))
        hot = np.concatenate([rng.choice(base, 2, replace=False), fresh[:2]])
        q = np.concatenate([np.repeat(hot[0], 1500), np.repeat(hot[1], 60),
                            np.repeat(hot[2], 900), np.repeat(hot[3], 40),
                            rng.choice(base, 900), rng.choice(fresh[2:], 900), crowd])
        q = q[rng.permutation(q.size)]
        _run(p, op if r else "find_or_insert", rng, q, strategy, dim, clock=50 + r,
             big=(r == 2))
