"""GPU parity: the gfx950 table, called through the C ABI, against the oracle.

Integer/byte results must be bit-exact: founds, returned rows, scores, the
full table contents exported in slot order (which pins slot placement and
eviction choices), evicted records (as multisets, their order is
unspecified in the reference) and sizes.  accum_or_assign's fp32 add is
also compared bit-exactly (one IEEE add per element, same operand order).
"""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, records_equal, to_dev, to_np
from helpers import keys_in_bucket, uniform_keys, values_for
from test_oracle import _strategy_case, _expected_epochlfu

pytestmark = pytest.mark.gpu


def rand_vals(rng, n, dim, dt=np.float32):
    if np.issubdtype(dt, np.floating):
        return rng.uniform(-1, 1, (n, dim)).astype(dt)
    info = np.iinfo(dt)
    return rng.integers(info.min, info.max, (n, dim), dtype=dt, endpoint=True)


def test_c1_plumbing_shape():
    """Customized, capacity 2^20, dim 16: fill to load factor 0.5 in 65,536-key
    batches, find 50% present / 50% absent, erase 10%, find again."""
    rng = np.random.default_rng(101)
    p = Pair(1 << 20, dim=16, strategy=O.CUSTOMIZED)
    allk = uniform_keys(rng, 8 * 65536)
    for b in range(8):
        ks = allk[b * 65536:(b + 1) * 65536]
        p.insert_or_assign(ks, rand_vals(rng, ks.size, 16),
                           rng.integers(0, 2**64 - 1, ks.size, dtype=np.uint64))
    p.assert_same_state()
    assert p.g.size() == 8 * 65536
    q = np.concatenate([rng.choice(allk, 32768, replace=False),
                        uniform_keys(rng, 32768, exclude=allk)])
    rng.shuffle(q)
    of = p.assert_same_find(q, fill=7)
    assert of.sum() == 32768
    er = rng.choice(allk, 52429, replace=False)
    p.erase(er)
    p.assert_same_state()
    assert p.g.size() == 8 * 65536 - 52429
    p.assert_same_find(q, fill=3)


@pytest.mark.parametrize("same_clock", [False, True])
def test_lru_fill_past_full(same_clock):
    """kLru from empty to well past load factor 1: placement, every eviction
    victim (including 16-lane tie-breaks when all clocks are equal) and
    scores match."""
    rng = np.random.default_rng(102 + same_clock)
    cap = 1 << 14
    p = Pair(cap, dim=8, strategy=O.LRU)
    for b in range(12):
        ks = uniform_keys(rng, 2048)
        p.insert_or_assign(ks, rand_vals(rng, 2048, 8),
                           clock=1000 if same_clock else 1000 + b)
        p.assert_same_state()
    assert p.g.load_factor() == 1.0


def test_fill_166_batches_to_full():
    """tests/test_insert_or_assign.cpp:170-228 on the GPU."""
    p = Pair(128 * 1024, dim=8, strategy=O.LRU)
    batches = 0
    while p.g.load_factor() != 1.0:
        ks = np.arange(1024 * batches, 1024 * (batches + 1), dtype=np.uint64)
        p.insert_or_assign(ks, values_for(ks, 8), clock=batches + 1)
        batches += 1
        assert batches <= 166
    assert batches == 166
    p.assert_same_state()


@pytest.mark.parametrize("strategy", [O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU,
                                      O.CUSTOMIZED])
def test_evict_strategy_basic(strategy):
    """tests/community/merlin_hashtable_test.cpp:1031-1306 on the GPU."""
    base, s_base, v_base, test, s_test, v_test = _strategy_case(strategy, 3)
    p = Pair(8 * 128, dim=4, strategy=strategy)
    no_sc = strategy in (O.LRU, O.EPOCH_LRU)
    clk1, clk2 = 1_000_000_000 << 20, 2_000_000_000 << 20
    p.set_global_epoch(1)
    p.insert_or_assign(base, v_base, None if no_sc else s_base, clock=clk1)
    p.assert_same_state()
    p.set_global_epoch(2)
    p.insert_or_assign(test, v_test, None if no_sc else s_test, clock=clk2)
    p.assert_same_state()
    assert p.g.size() == 128
    if strategy == O.EPOCH_LFU:
        (_, _, _), (gk, _, gs) = p.export()
        i71 = np.nonzero(gk == base[71])[0]
        assert i71.size == 1
        assert int(gs[i71[0]]) == _expected_epochlfu(2, int(s_base[71]) * 2)


@pytest.mark.parametrize("strategy", [O.CUSTOMIZED, O.LFU, O.EPOCH_LFU, O.LRU])
def test_duplicate_keys_non_unique(strategy):
    """unique_key=false with repeated keys in a batch, into a table that fills
    up: applied in batch order (32-lane find_and_lock tie-breaks)."""
    rng = np.random.default_rng(104)
    cap = 1 << 12
    p = Pair(cap, dim=4, strategy=strategy)
    p.set_global_epoch(5)
    pool = uniform_keys(rng, 6000)
    for b in range(6):
        ks = rng.choice(pool, 3000)
        sc = None if strategy == O.LRU else rng.integers(0, 50, ks.size, dtype=np.uint64)
        p.insert_or_assign(ks, rand_vals(rng, ks.size, 4), sc, unique_key=False,
                           clock=77 + b)
        p.assert_same_state()


def test_single_bucket_overflowing_pending_list():
    """1024 keys into a one-bucket table (tests/test_insert_or_assign.cpp:
    230-263): the bucket receives more keys than the pending list holds and
    takes the batch-walking path."""
    p = Pair(128, dim=8, strategy=O.LRU)
    ks = np.arange(1024, dtype=np.uint64)
    p.insert_or_assign(ks, values_for(ks, 8), clock=9)
    p.assert_same_state()
    assert p.g.size() == 128
    of = p.assert_same_find(ks)
    assert of.sum() == 128


def test_many_heavy_buckets():
    rng = np.random.default_rng(105)
    p = Pair(16 * 128, dim=2, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 5000)
    p.insert_or_assign(ks, rand_vals(rng, 5000, 2),
                       rng.integers(0, 1000, 5000, dtype=np.uint64))
    p.assert_same_state()
    p.insert_or_assign(ks[::-1].copy(), rand_vals(rng, 5000, 2),
                       rng.integers(0, 1000, 5000, dtype=np.uint64), unique_key=False)
    p.assert_same_state()


@pytest.mark.parametrize("strategy,unique", [(O.CUSTOMIZED, True), (O.LFU, True),
                                             (O.EPOCH_LFU, False), (O.LRU, False)])
def test_find_or_insert(strategy, unique):
    rng = np.random.default_rng(106)
    p = Pair(1 << 12, dim=8, strategy=strategy)
    p.set_global_epoch(3)
    pool = uniform_keys(rng, 8000)
    for b in range(5):
        ks = pool[rng.permutation(8000)[:2500]] if unique else rng.choice(pool, 2500)
        sc = None if strategy == O.LRU else rng.integers(1, 9, ks.size, dtype=np.uint64)
        ov, gv = p.find_or_insert(ks, rand_vals(rng, ks.size, 8), sc, unique,
                                  clock=100 + b)
        np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        p.assert_same_state()




@pytest.mark.parametrize("strategy,unique", [(O.CUSTOMIZED, True), (O.LFU, True),
                                             (O.CUSTOMIZED, False), (O.LRU, True)])
def test_insert_and_evict(strategy, unique):
    rng = np.random.default_rng(107)
    cap = 1 << 12
    p = Pair(cap, dim=16, strategy=strategy)
    pool = uniform_keys(rng, 12000)
    for b in range(6):
        sel = rng.permutation(12000)[:3000]
        ks = pool[sel] if unique else rng.choice(pool, 3000)
        sc = None if strategy == O.LRU else rng.integers(0, 100, ks.size, dtype=np.uint64)
        o, g = p.insert_and_evict(ks, rand_vals(rng, ks.size, 16), sc, unique,
                                  clock=500 + b)
        records_equal(o, g)
        p.assert_same_state()


def test_insert_and_evict_rejects_low_scores():
    """tests/test_insert_and_evict.cpp:679-745 on the GPU."""
    rng = np.random.default_rng(108)
    cap, dim = 4 * 128, 8
    p = Pair(cap, dim=dim, strategy=O.CUSTOMIZED)
    hi = keys_in_bucket(rng, 128, cap, 0, lo=1, hi=10_000_000)
    o, g = p.insert_and_evict(hi, values_for(hi, dim), np.arange(500, 628, dtype=np.uint64))
    assert g[0].size == 0
    lo = keys_in_bucket(rng, 64, cap, 0, lo=100_000_000, hi=200_000_000)
    o, g = p.insert_and_evict(lo, values_for(lo, dim), np.arange(64, dtype=np.uint64))
    assert g[0].size == 64
    records_equal(o, g)
    p.assert_same_state()


def test_accum_or_assign():
    rng = np.random.default_rng(109)
    p = Pair(1 << 12, dim=16, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 1500)
    p.insert_or_assign(ks, rand_vals(rng, 1500, 16),
                       rng.integers(0, 1000, 1500, dtype=np.uint64))
    for b in range(4):
        q = np.concatenate([rng.choice(ks, 700, replace=False), uniform_keys(rng, 700, exclude=ks)])
        flags = rng.integers(0, 2, q.size).astype(np.uint8)
        deltas = rng.uniform(-0.01, 0.01, (q.size, 16)).astype(np.float32)
        p.accum_or_assign(q, deltas, flags, rng.integers(0, 1000, q.size, dtype=np.uint64))
        p.assert_same_state()


@pytest.mark.parametrize("strategy", [O.CUSTOMIZED, O.LFU, O.LRU])
def test_accum_or_assign_repeated_keys(strategy):
    """accum_or_assign with keys repeated in a batch and mixed flags: an
    assign followed by accumulations of the same key, accumulations of one
    present key in a row, no-op flag mismatches, into a table that fills and
    evicts; i32 rows check the integer accumulation."""
    rng = np.random.default_rng(117)
    for vt, dt in (("f32", np.float32), ("i32", np.int32)):
        p = Pair(1 << 12, dim=8, strategy=strategy, vt=vt)
        pool = uniform_keys(rng, 3000)
        base = pool[:1500]
        init = (rand_vals(rng, base.size, 8) if vt == "f32"
                else rng.integers(-10**6, 10**6, (base.size, 8)).astype(np.int32))  # no overflow
        p.insert_or_assign(base, init, None if strategy == O.LRU else
                           rng.integers(0, 1000, base.size, dtype=np.uint64))
        for b in range(5):
            q = rng.choice(pool, 4000)
            flags = rng.integers(0, 2, q.size).astype(np.uint8)
            deltas = (rng.uniform(-0.01, 0.01, (q.size, 8)).astype(np.float32) if vt == "f32"
                      else rng.integers(-1000, 1000, (q.size, 8)).astype(np.int32))
            p.accum_or_assign(q, deltas, flags,
                              None if strategy == O.LRU else
                              rng.integers(0, 1000, q.size, dtype=np.uint64), clock=50 + b)
            p.assert_same_state()


def test_assign_scores():
    rng = np.random.default_rng(110)
    p = Pair(1 << 12, dim=4, strategy=O.LFU)
    ks = uniform_keys(rng, 1800)
    p.insert_or_assign(ks, rand_vals(rng, 1800, 4), rng.integers(0, 100, 1800, dtype=np.uint64))
    q = np.concatenate([rng.choice(ks, 900), uniform_keys(rng, 300, exclude=ks)])
    p.assign_scores(q, rng.integers(0, 100, q.size, dtype=np.uint64))
    p.assert_same_state()


def test_reserve_and_auto_growth():
    """reserve from load factor ~0.95 (rehash plus backward-shift
    defragmentation), then growth triggered by fast_load_factor."""
    rng = np.random.default_rng(111)
    p = Pair(1 << 12, 1 << 16, dim=8, strategy=O.CUSTOMIZED, max_load_factor=1.0)
    while p.g.size() < 3900:
        ks = uniform_keys(rng, 64)
        p.insert_or_assign(ks, rand_vals(rng, 64, 8),
                           rng.integers(0, 10**6, 64, dtype=np.uint64))
        assert p.g.capacity() == 1 << 12
    p.assert_same_state()
    p.reserve(1 << 14)
    assert p.g.capacity() == 1 << 14
    p.assert_same_state()
    q = Pair(1 << 12, 1 << 16, dim=8, strategy=O.CUSTOMIZED)
    for b in range(4):
        k2 = uniform_keys(rng, 3000)
        q.insert_or_assign(k2, rand_vals(rng, 3000, 8), rng.integers(0, 10**6, 3000, dtype=np.uint64))
        q.assert_same_state()
    assert q.g.capacity() > 1 << 12


def test_find_missed():
    rng = np.random.default_rng(112)
    p = Pair(1 << 14, dim=8, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 5000)
    p.insert_or_assign(ks, rand_vals(rng, 5000, 8), np.arange(5000, dtype=np.uint64))
    q = np.concatenate([ks[:2000], uniform_keys(rng, 1000, exclude=ks),
                        np.array([0xFFFFFFFFFFFFFFFF], np.uint64)])
    rng.shuffle(q)
    ov, omk, omi, _ = p.o.find_missed(q, np.zeros((q.size, 8), np.float32))
    torch = p.torch
    gv = to_dev(np.zeros((q.size, 8), np.float32))
    gmk = torch.zeros(q.size, dtype=torch.int64, device="cuda")
    gmi = torch.zeros(q.size, dtype=torch.int32, device="cuda")
    gms = torch.full((1,), 99, dtype=torch.int32, device="cuda")
    p.g.find_missed(q.size, to_dev(q), gv, gmk, gmi, gms)
    m = int(gms.item())
    assert m == omk.size == q.size - 2000
    gi = to_np(gmi, np.int32)[:m]
    gk = to_np(gmk, np.uint64)[:m]
    o = np.argsort(gi)
    np.testing.assert_array_equal(gi[o], omi)
    np.testing.assert_array_equal(gk[o], omk)
    np.testing.assert_array_equal(to_np(gv, np.float32).reshape(-1, 8), ov)


def test_reserved_keys_and_empty_batches():
    p = Pair(1 << 12, dim=4, strategy=O.CUSTOMIZED)
    ks = np.array([0xFFFFFFFFFFFFFFFF, 0xFFFFFFFFFFFFFFFE, 0xFFFFFFFFFFFFFFFD,
                   0xFFFFFFFFFFFFFFFC, 0, 1, 2], np.uint64)
    p.insert_or_assign(ks, np.ones((7, 4), np.float32), np.arange(7, dtype=np.uint64))
    p.assert_same_state()
    assert p.g.size() == 3
    p.assert_same_find(ks)
    e = np.zeros(0, np.uint64)
    p.g.insert_or_assign(0, None, None, None)
    p.g.find(0, None, None, None)
    p.g.erase(0, None)
    p.assert_same_state()


def test_every_batch_api_with_zero_keys():
    """n == 0 returns before any argument check, with null pointers, and
    leaves the table and the caller's counters alone
    (include/hkv_hashtable.h:1099, 1270, 2182); export_batch and
    export_batch_if still clear their counter first (:2530, :2636)."""
    import hkv_amd
    import torch
    rng = np.random.default_rng(115)
    p = Pair(1 << 12, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 1500)
    p.insert_or_assign(ks, rand_vals(rng, 1500, 4), rng.integers(1, 1000, 1500, dtype=np.uint64))
    g = p.g
    g.insert_or_assign(0, None, None, None)
    g.insert_or_assign_noalloc(0, None, None, None)
    cnt = torch.full((1,), 7, dtype=torch.int64, device="cuda")
    g.insert_and_evict(0, None, None, None, None, None, None, d_evicted_counter=cnt)
    assert g.insert_and_evict(0, None, None, None, None, None, None) == 0
    g.accum_or_assign(0, None, None, None, None)
    g.find_or_insert(0, None, None, None)
    g.find_or_insert(0, None, None, None, unique_key=False)
    g.assign_scores(0, None, None)
    g.assign(0, None, None, None)
    g.assign_values(0, None, None)
    g.contains(0, None, None)
    g.find(0, None, None, None)
    ms = torch.full((1,), 5, dtype=torch.int32, device="cuda")
    g.find_missed(0, None, None, None, None, ms)
    g.find_ptr(0, None, None)
    g.find_and_update(0, None, None)
    g.find_or_insert_ptr(0, None, None, None)
    g.lock_keys(0, None, None)
    g.unlock_keys(0, None, None)
    g.erase(0, None)
    ec = torch.full((1,), 9, dtype=torch.int64, device="cuda")
    g.export_batch(0, 0, None, None, None, d_counter=ec)
    ei = torch.full((1,), 9, dtype=torch.int64, device="cuda")
    g.export_batch_if(hkv_amd.PRED_SCORE_LT, 0, 0, 0, 0, ei, None, None)
    torch.cuda.synchronize()
    assert int(cnt.item()) == 7 and int(ms.item()) == 5
    assert int(ec.item()) == 0 and int(ei.item()) == 0
    assert g.size() == 1500
    p.assert_same_state()


@pytest.mark.parametrize("vt,dim", [("f32", 1), ("f32", 27), ("f32", 64),
                                    ("f32", 128), ("u8", 3), ("f16", 8),
                                    ("i64", 5), ("f64", 2)])
def test_row_sizes_and_value_types(vt, dim):
    rng = np.random.default_rng(113)
    from gpu_pair import NP_OF
    dt = NP_OF[vt]
    p = Pair(1 << 12, dim=dim, strategy=O.CUSTOMIZED, vt=vt)
    for b in range(3):
        ks = uniform_keys(rng, 2500)
        vals = (rng.integers(0, 255, (2500, dim)).astype(dt) if dt in (np.uint8,)
                else rand_vals(rng, 2500, dim, dt))
        p.insert_or_assign(ks, vals, rng.integers(0, 1000, 2500, dtype=np.uint64))
        p.assert_same_state()
        p.assert_same_find(np.concatenate([ks[:1000], uniform_keys(rng, 500)]))


def test_hybrid_host_values():
    """max_hbm_for_vectors below the value footprint: rows of the remaining
    buckets live in pinned host memory and are accessed in place."""
    rng = np.random.default_rng(114)
    dim = 64
    cap = 1 << 16
    p = Pair(cap, dim=dim, strategy=O.CUSTOMIZED, max_hbm=2 << 20)
    assert not p.g.is_pure_hbm_mode()
    for b in range(4):
        ks = uniform_keys(rng, 8192)
        p.insert_or_assign(ks, rand_vals(rng, 8192, dim), rng.integers(0, 1000, 8192, dtype=np.uint64))
    p.assert_same_state()
    p.assert_same_find(np.concatenate([ks, uniform_keys(rng, 1000)]))
    import hkv_amd
    with pytest.raises(RuntimeError):
        p.insert_and_evict(ks[:10], rand_vals(rng, 10, dim), np.arange(10, dtype=np.uint64))


def test_export_partial_ranges():
    rng = np.random.default_rng(115)
    p = Pair(1 << 12, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 1500)
    p.insert_or_assign(ks, rand_vals(rng, 1500, 4), rng.integers(0, 1000, 1500, dtype=np.uint64))
    for off, n in [(0, 1), (5, 300), (100, 1000), (4000, 500), (4096, 10), (0, 10**6)]:
        (ok, ov, os_), (gk, gv, gs) = p.export(n, off)
        np.testing.assert_array_equal(gk, ok)
        np.testing.assert_array_equal(gs, os_)
        np.testing.assert_array_equal(gv, ov)


def test_epoch_lru_epochs():
    rng = np.random.default_rng(116)
    p = Pair(1 << 11, dim=4, strategy=O.EPOCH_LRU)
    for e in range(6):
        p.set_global_epoch(e)
        ks = uniform_keys(rng, 1200)
        p.insert_or_assign(ks, rand_vals(rng, 1200, 4), clock=(e + 1) << 22)
        p.assert_same_state()


def test_argument_errors():
    import hkv_amd
    p = Pair(1 << 12, dim=4, strategy=O.LRU)
    ks = to_dev(np.arange(10, dtype=np.uint64))
    vs = to_dev(np.zeros((10, 4), np.float32))
    sc = to_dev(np.arange(10, dtype=np.uint64))
    with pytest.raises(hkv_amd.HkvException):
        p.g.insert_or_assign(10, ks, vs, sc)
    q = Pair(1 << 12, dim=4, strategy=O.EPOCH_LFU)
    with pytest.raises(hkv_amd.HkvException):
        q.g.insert_or_assign(10, ks, vs, sc)  # epoch never set
    r = Pair(1 << 12, dim=4, strategy=O.CUSTOMIZED)
    with pytest.raises(hkv_amd.HkvException):
        r.g.insert_or_assign(10, ks, vs, None)
