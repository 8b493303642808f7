"""GPU parity of erase_if / size_if / export_batch_if with the built-in
predicates of the C ABI, and of set_max_capacity, against the oracle.  The
functor forms of the C++ facade run in tests/cpp/facade_predicates.hip."""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, to_dev, to_np
from helpers import uniform_keys, values_for

pytestmark = pytest.mark.gpu

CASES = [(0, 0, 500), (1, 0, 500), (2, 0, 900), (3, 0x5, 0), (4, 0x3F, 300)]


def _rows(k, s, v):
    if k.size == 0:
        return np.zeros((0, 16 + np.asarray(v).itemsize * v.shape[-1]), np.uint8)
    a = np.concatenate([k.reshape(-1, 1).view(np.uint8), s.reshape(-1, 1).view(np.uint8),
                        np.ascontiguousarray(v).reshape(k.size, -1).view(np.uint8)], axis=1)
    return a[np.lexsort(a.T[::-1])] if a.size else a


@pytest.mark.parametrize("kind,pat,th", CASES)
@pytest.mark.parametrize("dim", [8, 3])
def test_predicates_match_oracle(kind, pat, th, dim):
    import torch
    rng = np.random.default_rng(50 + kind)
    p = Pair(1 << 13, dim=dim, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 3000)
    p.insert_or_assign(ks, values_for(ks, dim), rng.integers(0, 1000, size=ks.size,
                                                             dtype=np.uint64))
    cnt = torch.zeros(1, dtype=torch.int64, device="cuda")
    p.g.size_if(kind, pat, th, cnt)
    assert int(cnt.item()) == p.o.size_if(kind, pat, th)
    for n, off in [(1 << 13, 0), (2000, 3000), (100, (1 << 13) - 50), (10, 1 << 13)]:
        gk = torch.zeros(max(n, 1), dtype=torch.int64, device="cuda")
        gv = to_dev(np.zeros((max(n, 1), dim), np.float32))
        gs = torch.zeros(max(n, 1), dtype=torch.int64, device="cuda")
        p.g.export_batch_if(kind, pat, th, n, off, cnt, gk, gv, gs)
        c = int(cnt.item())
        ok, ov, os_ = p.o.export_batch_if(kind, pat, th, n, off)
        assert c == ok.size
        np.testing.assert_array_equal(
            _rows(to_np(gk, np.uint64)[:c], to_np(gs, np.uint64)[:c],
                  to_np(gv, np.float32).reshape(-1, dim)[:c]),
            _rows(ok, os_, ov))
    erased = p.g.erase_if(kind, pat, th)
    assert erased == p.o.erase_if(kind, pat, th)
    p.assert_same_state()
    p.assert_same_find(ks)


def test_predicates_hybrid_rows():
    # export_batch_if reads rows from pinned host slices; erase_if there
    import torch
    rng = np.random.default_rng(77)
    p = Pair(1 << 13, dim=8, strategy=O.CUSTOMIZED, max_hbm=(1 << 13) * 32 // 4)
    assert not p.g.is_pure_hbm_mode()
    ks = uniform_keys(rng, 3000)
    p.insert_or_assign(ks, values_for(ks, 8), rng.integers(0, 1000, size=ks.size,
                                                           dtype=np.uint64))
    cnt = torch.zeros(1, dtype=torch.int64, device="cuda")
    n = 1 << 13
    gk = torch.zeros(n, dtype=torch.int64, device="cuda")
    gv = to_dev(np.zeros((n, 8), np.float32))
    gs = torch.zeros(n, dtype=torch.int64, device="cuda")
    p.g.export_batch_if(1, 0, 400, n, 0, cnt, gk, gv, gs)
    c = int(cnt.item())
    ok, ov, os_ = p.o.export_batch_if(1, 0, 400, n, 0)
    assert c == ok.size > 0
    np.testing.assert_array_equal(
        _rows(to_np(gk, np.uint64)[:c], to_np(gs, np.uint64)[:c],
              to_np(gv, np.float32).reshape(-1, 8)[:c]), _rows(ok, os_, ov))
    assert p.g.erase_if(0, 0, 300) == p.o.erase_if(0, 0, 300)
    p.assert_same_state()


def test_signed_key_predicate():
    import torch
    import hkv_amd as H
    rng = np.random.default_rng(8)
    g = H.HashTable("i64", "f32", H.EvictStrategy.kCustomized)
    g.init(H.HashTableOptions(init_capacity=4096, max_capacity=4096,
                              max_hbm_for_vectors=1 << 40, dim=4))
    o = O.Oracle(4096, dim=4, strategy=O.CUSTOMIZED)
    ks = uniform_keys(rng, 1500)
    sc = rng.integers(0, 1000, size=ks.size, dtype=np.uint64)
    o.insert_or_assign(ks, values_for(ks, 4), sc)
    g.insert_or_assign(ks.size, to_dev(ks), to_dev(values_for(ks, 4)), to_dev(sc))
    # pattern -1 as int64: every (key & 0x7f) exceeds it, unlike the
    # unsigned reading
    pat = 0xFFFFFFFFFFFFFFFF
    e = g.erase_if(4, pat, 500)
    assert e == o.erase_if(4, pat, 500, key_signed=True) > 0
    assert g.size() == o.size()


def test_set_max_capacity_and_empty():
    import hkv_amd as H
    rng = np.random.default_rng(3)
    p = Pair(1024, 1024, dim=4, strategy=O.CUSTOMIZED)
    assert p.g.empty()
    with pytest.raises(H.UnsupportedError):
        p.g.set_max_capacity(3000)
    ks = uniform_keys(rng, 900)
    p.insert_or_assign(ks, values_for(ks, 4), np.ones(900, np.uint64))
    assert p.g.capacity() == 1024 and not p.g.empty()
    p.g.set_max_capacity(4096)
    p.o.set_max_capacity(4096)
    ks2 = uniform_keys(rng, 900, exclude=ks)
    p.insert_or_assign(ks2, values_for(ks2, 4), np.ones(900, np.uint64))
    assert p.g.capacity() == p.o.capacity() == 4096
    p.assert_same_state()
