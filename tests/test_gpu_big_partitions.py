"""GPU parity against the oracle for partitions (256 buckets) that receive
more than 4096 entries of a batch with repeated keys: their per-bucket
counts, heavy-bucket fold and per-occurrence row work run over the whole
GPU (k_big_count, k_big_fold, k_big_tasks) instead of in one block.

Covered: many such partitions in one call (Zipf batches over a small key
universe), each mutating operation with unique_key=false, every strategy,
and the cases the grid-wide path hands back to the block: a key map with
more than 1024 distinct keys, a heavy bucket whose new keys do not fit its
EMPTY slots, and more than 1024 entries in the other buckets.
"""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, records_equal
from helpers import keys_in_bucket, uniform_keys, zipf_keys

pytestmark = pytest.mark.gpu


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def scores(strategy, rng, n):
    if strategy in (O.LRU, O.EPOCH_LRU):
        return None
    return rng.integers(0, 1 << 34, n, dtype=np.uint64)


def run_op(p, op, rng, q, strategy, dim, clock):
    sc = scores(strategy, rng, q.size)
    v = rand_vals(rng, q.size, dim)
    if op == "find_or_insert":
        ov, gv = p.find_or_insert(q, v, sc, unique_key=False, clock=clock)
        np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    elif op == "insert_or_assign":
        p.insert_or_assign(q, v, sc, unique_key=False, clock=clock)
    elif op == "insert_and_evict":
        o, g = p.insert_and_evict(q, v, sc, unique_key=False, clock=clock)
        records_equal(o, g)
    else:
        p.assign_scores(q, sc, clock=clock)
    p.assert_same_state()


@pytest.mark.parametrize("op", ["find_or_insert", "insert_or_assign", "insert_and_evict",
                                "assign_scores"])
@pytest.mark.parametrize("strategy", [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU, O.CUSTOMIZED])
def test_zipf_batches_many_big_partitions(op, strategy):
    """2^20 slots (32 partitions) and 2^17-key Zipf(1.05) batches over 2^16
    keys: every partition gets about 4096 entries plus its hot keys, so many
    are big; the denser ones overflow the key map and go back to the block."""
    rng = np.random.default_rng(700 + strategy)
    cap, dim = 1 << 20, 4
    p = Pair(cap, dim=dim, strategy=strategy)
    for r in range(3):
        p.set_global_epoch(r)
        q = zipf_keys(rng, 1 << 17, universe=1 << 16)
        run_op(p, op if r else "find_or_insert", rng, q, strategy, dim, clock=100 + r)


def test_big_partition_fallbacks():
    """One partition (2^15 slots): a hot key 20,000 times with (a) 3000
    distinct keys twice each (heavy buckets with more than 1024 distinct keys
    in all: the map overflows), (b) 1600 light keys once each (more than 1024
    entries outside the heavy buckets), (c) a hot bucket whose 140 new keys
    exceed its EMPTY slots."""
    rng = np.random.default_rng(710)
    cap, dim = 1 << 15, 8
    hot = uniform_keys(rng, 1)
    for case in ("map_overflow", "many_light", "serial_bucket"):
        p = Pair(cap, dim=dim, strategy=O.LFU)
        base = uniform_keys(rng, 2000, exclude=hot)
        p.insert_or_assign(base, rand_vals(rng, base.size, dim),
                           scores(O.LFU, rng, base.size), clock=1)
        if case == "map_overflow":
            extra = np.repeat(uniform_keys(rng, 3000, exclude=base), 2)
        elif case == "many_light":
            extra = uniform_keys(rng, 1600, exclude=base)
        else:
            extra = np.repeat(keys_in_bucket(rng, 140, cap, 0, lo=1 << 40, hi=1 << 62), 3)
        q = np.concatenate([np.repeat(hot, 20000), extra])
        q = q[rng.permutation(q.size)]
        for r, op in enumerate(("find_or_insert", "insert_or_assign", "find_or_insert")):
            run_op(p, op, rng, q, O.LFU, dim, clock=10 + r)


def test_hot_keys_in_many_partitions_one_call():
    """Forty hot keys in different partitions of a 2^22-slot table (128
    partitions), 6000 occurrences each, plus uniform keys: forty big slots in
    one call, tiles of all of them interleaved over the grid."""
    rng = np.random.default_rng(720)
    cap, dim = 1 << 22, 4
    p = Pair(cap, dim=dim, strategy=O.EPOCH_LFU)
    p.set_global_epoch(7)
    hot = uniform_keys(rng, 40)
    for r in range(2):
        light = uniform_keys(rng, 60000, exclude=hot)
        q = np.concatenate([np.repeat(hot, 6000), light])
        q = q[rng.permutation(q.size)]
        run_op(p, "find_or_insert", rng, q, O.EPOCH_LFU, dim, clock=20 + r)
