"""GPU parity of each route through the partitioned apply pipeline.

A mutating batch is applied per partition (256 consecutive buckets):
  * the single-run kernel, one lane per bucket, when the partition's keys fit
    one LDS load (1024) and no bucket receives more than 32 of them;
  * the 16-lane kernel for buckets of that kernel that need eviction;
  * the multi-run kernel otherwise (large or skewed partitions);
  * row copies recorded per batch index and executed by a streaming kernel,
    with a later write of a row cancelling an earlier one and a
    find_or_insert hit on a row inserted earlier in the same batch reading
    that key's input.
Tables here have 512 or 1024 buckets so that batches of ~1000 keys take the
single-run route; the other GPU tests mostly use one-partition tables.
"""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, records_equal
from helpers import murmur3_np, uniform_keys

pytestmark = pytest.mark.gpu


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def keys_in_buckets(rng, n, capacity, b0, b1, exclude=()):
    """`n` distinct keys whose bucket lies in [b0, b1) (power-of-2 capacity)."""
    got, seen = [], set(int(x) for x in exclude)
    while len(got) < n:
        c = rng.integers(0, 2**63, size=1 << 18, dtype=np.uint64)
        b = (murmur3_np(c) & np.uint64(capacity - 1)) // np.uint64(128)
        for x in c[(b >= np.uint64(b0)) & (b < np.uint64(b1))]:
            if int(x) not in seen:
                seen.add(int(x))
                got.append(x)
                if len(got) == n:
                    break
    return np.array(got, np.uint64)


@pytest.mark.parametrize("strategy,same_clock", [(O.LRU, True), (O.LRU, False),
                                                 (O.CUSTOMIZED, False)])
def test_single_run_fill_past_full(strategy, same_clock):
    """~2 keys per bucket per batch into a 512-bucket table, from empty to
    well past full: lane pass, hand-over at the first eviction and the
    16-lane kernel."""
    rng = np.random.default_rng(301 + same_clock)
    cap = 1 << 16
    p = Pair(cap, dim=8, strategy=strategy)
    for b in range(90):
        ks = uniform_keys(rng, 1024)
        sc = None if strategy == O.LRU else rng.integers(0, 1 << 40, 1024, dtype=np.uint64)
        p.insert_or_assign(ks, rand_vals(rng, 1024, 8), sc,
                           clock=500 if same_clock else 500 + b)
        if b % 15 == 14 or b == 89:
            p.assert_same_state()
    assert p.g.load_factor() == 1.0


@pytest.mark.parametrize("strategy", [O.CUSTOMIZED, O.LRU])
def test_single_run_repeated_keys(strategy):
    """Batches drawn with replacement (unique_key=false): a row written twice
    in one batch keeps the later key's input."""
    rng = np.random.default_rng(303)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=strategy)
    pool = uniform_keys(rng, 40000)
    for b in range(30):
        ks = rng.choice(pool, 1024)
        sc = None if strategy == O.LRU else rng.integers(0, 100, 1024, dtype=np.uint64)
        p.insert_or_assign(ks, rand_vals(rng, 1024, 4), sc, unique_key=False, clock=9 + b)
        if b % 10 == 9:
            p.assert_same_state()
    p.assert_same_state()


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert"])
@pytest.mark.parametrize("strategy,scores,ignore", [
    (O.LRU, False, False), (O.LRU, True, True), (O.LFU, True, False),
    (O.EPOCH_LFU, True, False), (O.EPOCH_LFU, True, True), (O.EPOCH_LRU, False, False),
    (O.CUSTOMIZED, True, False)])
def test_single_run_repeat_fold(op, strategy, scores, ignore):
    """unique_key=false batches on the single-run route where keys repeat a
    few times inside a bucket: later occurrences are hits at the first one's
    slot, with the scores the sequential updates leave (EpochLfu inputs near
    2^31 saturate the low word).  The table fills to a load factor near 1.0,
    so repeats also fall past a bucket's first serial or evicting key."""
    rng = np.random.default_rng(305 + strategy)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=strategy)
    p.set_global_epoch(5)
    hot = uniform_keys(rng, 300)
    pool = uniform_keys(rng, 72000, exclude=hot)
    for b in range(90):
        ks = np.concatenate([rng.choice(hot, 256), pool[b * 800 + rng.permutation(800)[:768]]])
        ks = ks[rng.permutation(ks.size)]
        sc = None
        if scores:
            hi = (1 << 31) if strategy == O.EPOCH_LFU else (1 << 20)
            sc = rng.integers(1, hi, ks.size, dtype=np.uint64)
        v = rand_vals(rng, ks.size, 4)
        if op == "insert_or_assign":
            p.insert_or_assign(ks, v, sc, unique_key=False, ignore=ignore, clock=11 + b)
        else:
            ov, gv = p.find_or_insert(ks, v, sc, unique_key=False, ignore=ignore, clock=11 + b)
            np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        if b % 30 == 29:
            p.assert_same_state()
    assert p.g.load_factor() > 0.95


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert", "insert_and_evict"])
def test_single_run_new_keys_sharing_empty_slots(op):
    """Buckets filled to 100 of 128 slots, then batches of 8, 14 and 20 new
    keys per bucket on the single-run route: long runs of full slots make new keys
    of one call share their first EMPTY slot (a later key takes the next one
    its window recorded), run past the slots their window recorded (the
    serial lane), and fill buckets (the eviction kernel)."""
    rng = np.random.default_rng(306)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=O.LRU)
    buckets = list(range(0, 512, 11))  # at most 24 per partition
    fill = np.concatenate([keys_in_buckets(rng, 100, cap, b, b + 1) for b in buckets])
    p.insert_or_assign(fill, rand_vals(rng, fill.size, 4), None, clock=3)
    p.assert_same_state()
    for r in range(3):
        new = np.concatenate([keys_in_buckets(rng, 8 + 6 * r, cap, b, b + 1, exclude=fill)
                              for b in buckets])
        fill = np.concatenate([fill, new])
        q = np.concatenate([new, rng.choice(fill, 200)])
        q = q[rng.permutation(q.size)]
        v = rand_vals(rng, q.size, 4)
        if op == "insert_or_assign":
            p.insert_or_assign(q, v, None, unique_key=False, clock=10 + r)
        elif op == "find_or_insert":
            ov, gv = p.find_or_insert(q, v, None, unique_key=False, clock=10 + r)
            np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        else:
            o, g = p.insert_and_evict(q, v, None, unique_key=False, clock=10 + r)
            records_equal(o, g)
        p.assert_same_state()


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert"])
@pytest.mark.parametrize("strategy", [O.LFU, O.EPOCH_LFU, O.CUSTOMIZED])
def test_single_run_key_repeated_up_to_32(op, strategy):
    """A key repeated 20 to 32 times in one bucket of the single-run route
    (at most 32 keys per bucket, so no long-bucket split): the fold of its
    scores (EpochLfu inputs near 2^31 saturate the low word) and its rows,
    new and present keys, against the oracle."""
    rng = np.random.default_rng(308 + strategy)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=strategy)
    p.set_global_epoch(4)
    present = uniform_keys(rng, 2000)
    p.insert_or_assign(present, rand_vals(rng, present.size, 4),
                       rng.integers(1, 1 << 20, present.size, dtype=np.uint64), clock=2)
    for r in range(4):
        hot = np.concatenate([rng.choice(present, 6, replace=False),
                              uniform_keys(rng, 6, exclude=present)])
        reps = rng.integers(20, 33, hot.size)
        q = np.concatenate([np.repeat(hot, reps), rng.choice(present, 300),
                            uniform_keys(rng, 200, exclude=np.concatenate([present, hot]))])
        q = q[rng.permutation(q.size)]
        hi = (1 << 31) if strategy == O.EPOCH_LFU else (1 << 20)
        sc = rng.integers(1, hi, q.size, dtype=np.uint64)
        v = rand_vals(rng, q.size, 4)
        if op == "insert_or_assign":
            p.insert_or_assign(q, v, sc, unique_key=False, clock=20 + r)
        else:
            ov, gv = p.find_or_insert(q, v, sc, unique_key=False, clock=20 + r)
            np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        p.assert_same_state()
        present = np.unique(np.concatenate([present, q]))


@pytest.mark.parametrize("op", ["assign_scores", "insert_and_evict", "accum_or_assign"])
@pytest.mark.parametrize("strategy", [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU, O.CUSTOMIZED])
def test_single_run_full_buckets(op, strategy):
    """assign_scores, insert_and_evict and accum_or_assign on a table filled
    past full, on the single-run route: present keys anywhere in their
    bucket (also past the probe window and in the start chunk's groups
    before the start) are applied there, absent keys are no-ops
    (assign_scores, accumulations) or take the eviction path."""
    rng = np.random.default_rng(309 + strategy)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=strategy)
    p.set_global_epoch(3)
    uses = strategy not in (O.LRU, O.EPOCH_LRU)
    keys = uniform_keys(rng, 90000)
    for b in range(0, keys.size, 9000):
        ks = keys[b:b + 9000]
        p.insert_or_assign(ks, rand_vals(rng, ks.size, 4),
                           rng.integers(1, 1 << 30, ks.size, dtype=np.uint64) if uses else None,
                           clock=5 + b)
    p.assert_same_state()
    for r in range(3):
        q = np.concatenate([rng.choice(keys, 600, replace=False),
                            uniform_keys(rng, 600, exclude=keys)])
        q = q[rng.permutation(q.size)]
        sc = rng.integers(1, 1 << 31, q.size, dtype=np.uint64) if uses else None
        if op == "assign_scores":
            p.assign_scores(q, sc, clock=100 + r)
        elif op == "insert_and_evict":
            o, g = p.insert_and_evict(q, rand_vals(rng, q.size, 4), sc, clock=100 + r)
            records_equal(o, g)
        else:
            flags = np.isin(q, keys)
            flags[rng.random(q.size) < 0.2] ^= True  # some flags do not match
            p.accum_or_assign(q, rand_vals(rng, q.size, 4) * 0.01, flags, sc, clock=100 + r)
        p.assert_same_state()


@pytest.mark.parametrize("n", [8 * 1024, 9 * 1024 + 37, 17 * 1024 - 5])
def test_chunk_counts_around_the_xcd_mapping(n):
    """Batch chunks (1024 keys) are counted and scattered by blocks that take
    contiguous chunk ranges per XCD for the first 8 * floor(chunks / 8)
    chunks and their own index after that: batches of 8, 10 and 17 chunks,
    inserted and then found, against the oracle."""
    rng = np.random.default_rng(307)
    cap = 1 << 17
    p = Pair(cap, dim=4, strategy=O.CUSTOMIZED)
    for r in range(3):
        ks = uniform_keys(rng, n)
        sc = rng.integers(0, 1 << 30, n, dtype=np.uint64)
        p.insert_or_assign(ks, rand_vals(rng, n, 4), sc, clock=5 + r)
        ov, gv = p.find_or_insert(ks[rng.permutation(n)], rand_vals(rng, n, 4),
                                  rng.integers(0, 1 << 30, n, dtype=np.uint64), clock=9 + r)
        np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        p.assert_same_state()


@pytest.mark.parametrize("unique", [True, False])
def test_single_run_find_or_insert_reads_same_batch_rows(unique):
    """find_or_insert with keys repeated in a batch: the later occurrences
    return the row the first one inserted (copied from its input)."""
    rng = np.random.default_rng(304)
    cap = 1 << 16
    p = Pair(cap, dim=8, strategy=O.CUSTOMIZED)
    pool = uniform_keys(rng, 30000)
    for b in range(40):
        if unique:
            ks = rng.choice(pool, 1024, replace=False)
        else:
            ks = rng.choice(pool, 1024)
        sc = rng.integers(0, 1 << 20, ks.size, dtype=np.uint64)
        ov, gv = p.find_or_insert(ks, rand_vals(rng, ks.size, 8), sc, unique_key=unique,
                                  clock=3 + b)
        np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        if b % 10 == 9:
            p.assert_same_state()


def test_single_run_insert_and_evict_and_assign_scores():
    rng = np.random.default_rng(305)
    cap = 1 << 16
    p = Pair(cap, dim=4, strategy=O.LFU)
    pool = uniform_keys(rng, 120000)
    for b in range(80):
        ks = pool[1024 * b:1024 * (b + 1)] if b % 2 == 0 else rng.choice(pool[:1024 * b], 1024,
                                                                          replace=False)
        sc = rng.integers(0, 1 << 20, 1024, dtype=np.uint64)
        o, g = p.insert_and_evict(ks, rand_vals(rng, 1024, 4), sc, clock=b)
        records_equal(o, g)
        if b % 8 == 7:
            p.assign_scores(rng.choice(pool[:1024 * (b + 1)], 1024, replace=False),
                            rng.integers(0, 1 << 10, 1024, dtype=np.uint64))
            p.assert_same_state()
    p.assert_same_state()


def test_mixed_routes_in_one_call():
    """One batch whose partitions take all three routes: partition 0 has a
    bucket with 40 keys, partition 2 receives 1100 keys, partitions 1 and 3
    take the single-run kernel."""
    rng = np.random.default_rng(306)
    cap = 1 << 17  # 1024 buckets, 4 partitions
    p = Pair(cap, dim=4, strategy=O.CUSTOMIZED)
    for b in range(6):
        heavy = keys_in_buckets(rng, 40, cap, 3, 4)
        big = keys_in_buckets(rng, 1100, cap, 512, 768, exclude=heavy)
        rest = np.concatenate([keys_in_buckets(rng, 300, cap, 256, 512),
                               keys_in_buckets(rng, 300, cap, 768, 1024)])
        ks = np.concatenate([heavy, big, rest])
        rng.shuffle(ks)
        p.insert_or_assign(ks, rand_vals(rng, ks.size, 4),
                           rng.integers(0, 1 << 30, ks.size, dtype=np.uint64))
        p.assert_same_state()
        p.assert_same_find(ks)


@pytest.mark.parametrize("op", ["insert_or_assign", "find_or_insert"])
@pytest.mark.parametrize("per_bucket,new_frac", [(1.5, 0.5), (2.5, 0.8)])
def test_serial_bucket_rows_on_a_full_table(op, per_bucket, new_frac):
    """A full 512-bucket table and batches of resident and new keys: every
    bucket with a new key stops at it and hands the rest over, so the rows
    of the resident keys before the stop are copied after the block barrier,
    from the list of the serial buckets' row tasks (at 2.5 keys per bucket,
    4 in 5 of them new, over 192 of a block's 256 buckets stop, every wave
    holds serial lanes, and the block's last pass copies every row)."""
    rng = np.random.default_rng(331 + int(per_bucket * 10))
    cap, dim = 1 << 16, 32
    p = Pair(cap, dim=dim, strategy=O.CUSTOMIZED)
    resident = np.empty(0, np.uint64)
    while p.g.load_factor() < 1.0:
        ks = uniform_keys(rng, 2048, exclude=resident)
        p.insert_or_assign(ks, rand_vals(rng, 2048, dim),
                           rng.integers(1 << 20, 1 << 30, 2048, dtype=np.uint64))
        resident = np.concatenate([resident, ks])
    p.assert_same_state()
    (gk, _, _), _ = p.export()
    for b in range(3):
        n = int(512 * per_bucket)
        n_new = int(n * new_frac)
        live = rng.choice(gk, n - n_new, replace=False)
        new = uniform_keys(rng, n_new, exclude=resident)
        resident = np.concatenate([resident, new])
        ks = np.concatenate([live, new])
        rng.shuffle(ks)
        sc = rng.integers(1 << 30, 1 << 40, ks.size, dtype=np.uint64)
        if op == "insert_or_assign":
            p.insert_or_assign(ks, rand_vals(rng, ks.size, dim), sc)
        else:
            ov, gv = p.find_or_insert(ks, rand_vals(rng, ks.size, dim), sc)
            np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        p.assert_same_state()
        (gk, _, _), _ = p.export()


def test_batches_over_2_20_keys():
    """2^20 + 4096 keys per batch: 1028 chunks of 1024 keys, so the segment
    scan keeps a column's counts in memory rather than in registers (more
    than 32 chunks per thread); 8,000 entries per partition of a 2^23-slot
    table take the multi-run kernel."""
    rng = np.random.default_rng(341)
    cap, dim, n = 1 << 23, 4, (1 << 20) + 4096
    p = Pair(cap, dim=dim, strategy=O.CUSTOMIZED)
    seen = np.empty(0, np.uint64)
    for b in range(2):
        ks = uniform_keys(rng, n, exclude=seen if b else None)
        seen = np.concatenate([seen, ks])
        p.insert_or_assign(ks, rand_vals(rng, n, dim),
                           rng.integers(0, 1 << 40, n, dtype=np.uint64))
        p.assert_same_state()
    q = np.concatenate([rng.choice(seen, 4096, replace=False), uniform_keys(rng, 4096, exclude=seen)])
    of = p.assert_same_find(q)
    assert of.sum() == 4096
