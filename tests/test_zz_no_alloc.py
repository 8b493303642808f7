"""hkv_insert_or_assign_noalloc, called through the C ABI, against
hkv_insert_or_assign on a twin table fed the same batches.

The allocation-free entry point keeps its partition scratch in the
library's static device array instead of handle-owned buffers, so each
check compares full slot-ordered exports (keys, row bytes, scores) of the
two tables, bit-exactly, after every call.  Successive calls reuse the same
array: the second call of each sequence is smaller than the first, so a
region it reads must not keep the first call's contents.  The paths covered
are the single-run fast kernel, the eviction hand-over, the multi-run
partition kernel (partitions over 704 entries) and repeated keys; the error
cases are a batch whose scratch exceeds the array and a table below its
maximum capacity.
"""
import numpy as np
import pytest

import oracle as O
from gpu_pair import to_dev, to_np
from helpers import uniform_keys_fast

pytestmark = pytest.mark.gpu


def make(cap, dim, strategy, max_cap=None):
    import hkv_amd
    t = hkv_amd.HashTable("u64", "f32", strategy)
    t.init(hkv_amd.HashTableOptions(init_capacity=cap, max_capacity=max_cap or cap,
                                    max_hbm_for_vectors=1 << 40, dim=dim))
    return t


def export(t, dim):
    import torch
    cap = t.capacity()
    k = torch.zeros(cap, dtype=torch.int64, device="cuda")
    v = torch.zeros((cap, dim), dtype=torch.float32, device="cuda")
    s = torch.zeros(cap, dtype=torch.int64, device="cuda")
    c = t.export_batch(cap, 0, k, v, s)
    return (to_np(k, np.uint64)[:c], to_np(v, np.uint32).reshape(cap, dim)[:c],
            to_np(s, np.uint64)[:c])


def same(a, b, dim):
    assert a.size() == b.size()
    for x, y in zip(export(a, dim), export(b, dim)):
        np.testing.assert_array_equal(y, x)


def run_pair(cap, dim, strategy, sizes, seed, mix_max=1 << 30):
    """Feeds both tables the same batches of the given sizes; batches after
    the first of at most `mix_max` keys revisit the previous batch's keys
    and repeat keys (unique_key=False)."""
    rng = np.random.default_rng(seed)
    ref, na = make(cap, dim, strategy), make(cap, dim, strategy)
    if strategy == O.LRU:
        ref.set_lru_clock(4242)
        na.set_lru_clock(4242)
    prev = None
    for j, n in enumerate(sizes):
        ks = uniform_keys_fast(rng, n)
        unique = True
        if prev is not None and n <= mix_max:
            m = n // 3
            ks[:m] = rng.choice(prev, m)          # resident keys
            ks[m:m + m // 2] = ks[:m // 2]         # repeated keys
            unique = False
        vs = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
        sc = None if strategy == O.LRU else rng.integers(1, 1 << 40, n, dtype=np.uint64)
        kd, vd = to_dev(ks), to_dev(vs)
        sd = None if sc is None else to_dev(sc)
        ref.insert_or_assign(n, kd, vd, sd, 0, unique)
        na.insert_or_assign_noalloc(n, kd, vd, sd, 0, unique)
        same(ref, na, dim)
        prev = ks
    return ref, na


def test_noalloc_multi_run_partitions_and_eviction():
    """2^17 slots (4 partitions): a 2^16-key batch puts 16384 entries in each
    partition (the multi-run kernel), the 3000-key batch repeats and revisits
    keys, the later batches push the table past full (eviction)."""
    ref, na = run_pair(1 << 17, 16, O.CUSTOMIZED,
                       [1 << 16, 3000, 1 << 15, 1 << 16, 1 << 16], 11)
    assert na.size() == ref.size() and na.load_factor() > 0.9


def test_noalloc_fast_path_then_smaller_batch():
    """2^20 slots (32 partitions): 2^18-key batches of new keys fill it past
    a load factor of 0.9 through the multi-run kernel, then batches of at most 16384 keys
    (512 per partition) take the single-run fast kernel, whose full buckets
    go to the eviction hand-over."""
    ref, na = run_pair(1 << 20, 8, O.LRU,
                       [1 << 18, 1000, 1 << 18, 1 << 18, 1 << 18, 16384, 16384, 12000, 16384],
                       12, mix_max=20000)
    assert ref.load_factor() > 0.9


def test_noalloc_rejects_what_it_cannot_serve():
    import torch
    import hkv_amd
    # A 2^20-key batch on a 2^26-slot table needs ~88 MiB of scratch.
    t = make(1 << 26, 1, O.CUSTOMIZED)
    n = 1 << 20
    kd = to_dev(uniform_keys_fast(np.random.default_rng(13), n))
    vd = torch.zeros((n, 1), dtype=torch.float32, device="cuda")
    sd = torch.ones(n, dtype=torch.int64, device="cuda")
    with pytest.raises(hkv_amd.HkvException, match="MiB of scratch"):
        t.insert_or_assign_noalloc(n, kd, vd, sd)
    assert t.size() == 0
    t.insert_or_assign_noalloc(1 << 18, kd, vd, sd)  # a quarter of it fits
    assert t.size() == 1 << 18
    del t
    # A table that can still grow would allocate.
    g = make(1 << 14, 4, O.CUSTOMIZED, max_cap=1 << 16)
    k = to_dev(uniform_keys_fast(np.random.default_rng(14), 100))
    with pytest.raises(hkv_amd.HkvException, match="maximum capacity"):
        g.insert_or_assign_noalloc(100, k, torch.zeros((100, 4), device="cuda"),
                                   torch.ones(100, dtype=torch.int64, device="cuda"))
    assert g.size() == 0
