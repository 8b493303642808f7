"""GPU parity against the oracle at table shapes the power-of-two tests do
not reach.

* Bucket counts that are not powers of two.  When 2 * init_capacity >
  max_capacity the reference allocates ceil(max_capacity / 128) buckets
  (include/table.h:299-311), so `h mod capacity` takes the magic-number
  divide of include/utils.h:86-97 and include/table.h:106-127.
* Growth from such a table once set_max_capacity lifts the limit
  (include/hkv_hashtable.h:2955-2977): the last, short value slice is
  replaced by a longer one before the new buckets get theirs, in HBM and in
  pinned host memory.
* Multi-pass partition counting.  Tables with more partitions (256 buckets
  each) than the counting kernels' LDS histogram holds (16384, i.e. 2^29
  slots) are counted and scattered in several passes over each 1024-key
  chunk; HKV_PART_RANGE shrinks the histogram so that small tables take
  that path here.
"""
import numpy as np
import pytest

import oracle as O
import gpu_pair
from gpu_pair import Pair, records_equal
from helpers import uniform_keys, zipf_keys

pytestmark = pytest.mark.gpu


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def exercise(p, rng, n, rounds, dim, strategy):
    """Every mutating op plus find and erase, with duplicates, past full."""
    sc = (lambda m: rng.integers(1, 1 << 40, m, dtype=np.uint64)) \
        if strategy not in (O.LRU, O.EPOCH_LRU) else (lambda m: None)
    resident = np.empty(0, np.uint64)
    for r in range(rounds):
        if strategy in (O.EPOCH_LRU, O.EPOCH_LFU):
            p.set_global_epoch(r)
        ks = uniform_keys(rng, n)
        if resident.size:
            ks[: n // 4] = rng.choice(resident, n // 4)
        p.insert_or_assign(ks, rand_vals(rng, n, dim), sc(n), clock=100 + r)
        p.assert_same_state()
        dup = np.concatenate([ks[: n // 2], ks[: n // 8]])
        rng.shuffle(dup)
        ov, gv = p.find_or_insert(dup, rand_vals(rng, dup.size, dim), sc(dup.size),
                                  unique_key=False, clock=200 + r)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
        if p.g.is_pure_hbm_mode():  # the reference refuses it on hybrid tables
            o, g = p.insert_and_evict(uniform_keys(rng, n // 2), rand_vals(rng, n // 2, dim),
                                      sc(n // 2), clock=300 + r)
            records_equal(o, g)
        (resident, _, _), _ = p.export()
        q = np.concatenate([rng.choice(resident, n // 4), uniform_keys(rng, n // 4)])
        flags = (rng.random(q.size) < 0.5).astype(np.uint8)
        p.accum_or_assign(q, rng.uniform(-0.01, 0.01, (q.size, dim)).astype(np.float32),
                          flags, sc(q.size), clock=400 + r)
        p.assign_scores(rng.choice(resident, n // 4), sc(n // 4), clock=500 + r)
        p.assert_same_state()
        p.assert_same_find(np.concatenate([rng.choice(resident, n // 4),
                                           uniform_keys(rng, n // 4)]))
        p.erase(rng.choice(resident, n // 16))
        p.assert_same_state()
        (resident, _, _), _ = p.export()


@pytest.mark.parametrize("cap,strategy", [(3 << 14, O.CUSTOMIZED), (100_000, O.LFU),
                                          (1_000_003, O.EPOCH_LFU), (100_000, O.LRU)])
def test_general_capacity_matches_oracle(cap, strategy):
    rng = np.random.default_rng(cap % 997 + strategy)
    p = Pair(cap, dim=8, strategy=strategy)
    assert p.g.capacity() == p.o.capacity() == -(-cap // 128) * 128
    assert p.g.capacity() & (p.g.capacity() - 1)  # not a power of two
    n = max(1024, cap // 8)
    exercise(p, rng, n, 5, 8, strategy)
    assert p.g.size() == p.o.size()
    for off, n in ((0, 1000), (cap // 3, 4097), (p.g.capacity() - 100, 4096)):
        o, g = p.export(n, off)
        for a, b in zip(o, g):
            np.testing.assert_array_equal(b, a)


@pytest.mark.parametrize("hybrid", [False, True])
def test_growth_from_general_capacity(hybrid):
    """init = max = 100,000 slots (782 buckets), then set_max_capacity(2^18):
    inserts grow the table to 1564 buckets (200,192 slots).  With `hybrid`
    the value budget holds one 512-bucket slice, so the short slice being
    replaced and the new ones are pinned host memory."""
    rng = np.random.default_rng(77 + hybrid)
    dim = 8
    p = Pair(100_000, dim=dim, strategy=O.CUSTOMIZED,
             max_hbm=(512 * 128 * dim * 4) if hybrid else None)
    if hybrid:
        assert not p.g.is_pure_hbm_mode()
    ks = uniform_keys(rng, 40_000)
    p.insert_or_assign(ks, rand_vals(rng, ks.size, dim),
                       rng.integers(1, 1 << 40, ks.size, dtype=np.uint64))
    p.assert_same_state()
    for t in (p.o, p.g):
        t.set_max_capacity(1 << 18)
    assert p.g.capacity() == 782 * 128
    more = uniform_keys(rng, 60_000, exclude=ks)
    p.insert_or_assign(more, rand_vals(rng, more.size, dim),
                       rng.integers(1, 1 << 40, more.size, dtype=np.uint64))
    assert p.g.capacity() == p.o.capacity() == 1564 * 128
    p.assert_same_state()
    p.assert_same_find(np.concatenate([ks, more, uniform_keys(rng, 5000)]))
    exercise(p, rng, 8192, 2, dim, O.CUSTOMIZED)
    assert p.g.capacity() == 1564 * 128  # 2 * 200,192 > 2^18: at max capacity


@pytest.mark.parametrize("prange", [1, 3, 7])
def test_multi_pass_partition_counting(monkeypatch, prange):
    """2^20 slots = 32 partitions counted `prange` at a time (the last pass
    short when prange does not divide 32), with uniform and Zipf batches."""
    monkeypatch.setenv("HKV_PART_RANGE", str(prange))
    rng = np.random.default_rng(500 + prange)
    p = Pair(1 << 20, dim=4, strategy=O.LFU)
    exercise(p, rng, 1 << 15, 3, 4, O.LFU)
    for _ in range(3):
        ks = zipf_keys(rng, 1 << 15)
        ov, gv = p.find_or_insert(ks, rand_vals(rng, ks.size, 4),
                                  np.ones(ks.size, np.uint64), unique_key=False)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    p.assert_same_state()


def test_auto_grow_decisions_small_batches():
    """Auto-grow with batches of 1-300 keys (include/hkv_hashtable.h:
    1103-1106).  The table keeps a host-side upper bound on the sampled
    bucket sizes and synchronises for the exact sum only when the bound could
    cross max_load_factor; the capacity after every call must still be the
    oracle's.  Erases, a clear, a reserve and calls on a second stream (which
    turn the bound off) are mixed in."""
    rng = np.random.default_rng(91)
    dim = 4
    p = Pair(1024, max_capacity=1 << 16, dim=dim, strategy=O.LFU)
    torch = p.torch
    resident = np.empty(0, np.uint64)
    side = torch.cuda.Stream()
    for step in range(700):
        n = int(rng.integers(1, 301))
        ks = uniform_keys(rng, n)
        v = rand_vals(rng, n, dim)
        sc = rng.integers(1, 1 << 40, n, dtype=np.uint64)
        if step < 600:
            if step % 3 == 0:
                p.find_or_insert(ks, v, sc)
            else:
                p.insert_or_assign(ks, v, sc)
        else:
            p.o.insert_or_assign(ks, v, sc, True, False, 12345)
            with torch.cuda.stream(side):
                kd, vd, sd = gpu_pair.to_dev(ks), gpu_pair.to_dev(v), gpu_pair.to_dev(sc)
                p.g.insert_or_assign(n, kd, vd, sd, side.cuda_stream, True, False)
            side.synchronize()
        resident = np.concatenate([resident, ks])
        if step % 50 == 49:
            gone = rng.choice(resident, resident.size // 3, replace=False)
            p.erase(gone)
            resident = np.setdiff1d(resident, gone)
        if step == 300:
            p.clear()
            resident = np.empty(0, np.uint64)
        if step == 450:
            p.reserve(p.g.capacity() * 2)
        assert p.g.capacity() == p.o.capacity(), step
    p.assert_same_state()
