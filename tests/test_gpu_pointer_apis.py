"""GPU parity of the pointer APIs: find / find_or_insert pointer overloads,
find_and_update, lock_keys and unlock_keys, against the oracle.

The oracle returns slot indices; the library's addresses of those slots come
from hkv_slot_addresses, so every returned pointer is checked for the exact
slot, and the table layout afterwards (the slot of every key, its score) is
checked through the pointer find.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from gpu_pair import to_dev, to_np
from helpers import keys_in_bucket, uniform_keys, values_for

pytestmark = pytest.mark.gpu

NO = O.NO_SLOT
LOCKED = 0xFFFFFFFFFFFFFFFD
RESERVED = np.array([0xFFFFFFFFFFFFFFFF, 0xFFFFFFFFFFFFFFFE, 0xFFFFFFFFFFFFFFFC],
                    np.uint64)


def _mods():
    import torch
    import hkv_amd
    return torch, hkv_amd


def _hip():
    """The HIP runtime this process already uses (torch's bundled copy)."""
    with open("/proc/self/maps") as f:
        paths = [ln.split()[-1] for ln in f if "libamdhip64" in ln]
    lib = ctypes.CDLL(paths[0])
    lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                              ctypes.c_int]
    lib.hipMemcpy.restype = ctypes.c_int
    return lib


def read_rows(ptrs, row_bytes):
    """Rows at device-accessible addresses, one hipMemcpy each."""
    hip = _hip()
    out = np.zeros((len(ptrs), row_bytes), np.uint8)
    for i, p in enumerate(ptrs):
        assert hip.hipMemcpy(out[i].ctypes.data, int(p), row_bytes, 4) == 0
    return out


def write_rows(ptrs, rows):
    hip = _hip()
    rows = np.ascontiguousarray(rows)
    for i, p in enumerate(ptrs):
        assert hip.hipMemcpy(int(p), rows[i].ctypes.data, rows[i].nbytes, 4) == 0


def make(strategy, cap, max_cap=None, dim=8, max_hbm=1 << 40):
    torch, H = _mods()
    g = H.HashTable("u64", "f32", strategy)
    g.init(H.HashTableOptions(init_capacity=cap, max_capacity=max_cap or cap,
                              max_hbm_for_vectors=max_hbm, dim=dim))
    o = O.Oracle(cap, max_cap or cap, dim=dim, strategy=strategy)
    return g, o


def insert_both(g, o, ks, dim, scores=None, clock=100):
    v = values_for(ks, dim)
    o.insert_or_assign(ks, v, scores, clock=clock)
    g.set_lru_clock(clock)
    g.insert_or_assign(ks.size, to_dev(ks), to_dev(v),
                       None if scores is None else to_dev(scores))


def expected_ptrs(g, slots):
    """(key word, value row) addresses of oracle slots; 0 where NO_SLOT."""
    kp = np.zeros(slots.size, np.uint64)
    vp = np.zeros(slots.size, np.uint64)
    m = slots != NO
    if m.any():
        k, v = g.slot_addresses(slots[m])
        kp[m], vp[m] = k, v
    return kp, vp


def find_ptr_both(g, o, q):
    torch, _ = _mods()
    n = q.size
    vp = torch.zeros(n, dtype=torch.int64, device="cuda")
    fd = torch.zeros(n, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(n, dtype=torch.int64, device="cuda")
    g.find_ptr(n, to_dev(q), vp, fd, sc)
    torch.cuda.synchronize()
    oslots, ofound, oscores = o.find_ptr(q, with_scores=True)
    return (to_np(vp, np.uint64), to_np(fd, np.uint8).astype(bool),
            to_np(sc, np.uint64), oslots, ofound, oscores)


def assert_same_layout(g, o, keys):
    """Every key at the oracle's slot with the oracle's score."""
    vp, fd, sc, oslots, ofound, oscores = find_ptr_both(g, o, keys)
    np.testing.assert_array_equal(fd, ofound)
    np.testing.assert_array_equal(vp, expected_ptrs(g, oslots)[1])
    np.testing.assert_array_equal(sc[fd], oscores[ofound])
    assert g.size() == o.size()


@pytest.mark.parametrize("hybrid", [False, True])
def test_find_ptr_matches_oracle(hybrid):
    torch, H = _mods()
    rng = np.random.default_rng(1)
    dim = 8
    cap = 1 << 14
    # hybrid: a quarter of the rows in HBM, the rest in pinned host memory
    g, o = make(H.EvictStrategy.kCustomized, cap, dim=dim,
                max_hbm=(cap * dim * 4) // 4 if hybrid else 1 << 40)
    if hybrid:
        assert not g.is_pure_hbm_mode()
    ks = uniform_keys(rng, 6000)
    insert_both(g, o, ks, dim, rng.integers(1, 1 << 40, size=ks.size, dtype=np.uint64))
    q = np.concatenate([ks[:3000], uniform_keys(rng, 1000, exclude=ks), RESERVED])
    vp, fd, sc, oslots, ofound, oscores = find_ptr_both(g, o, q)
    np.testing.assert_array_equal(fd, ofound)
    np.testing.assert_array_equal(vp, expected_ptrs(g, oslots)[1])
    assert np.all(vp[~fd] == 0)
    np.testing.assert_array_equal(sc[fd], oscores[ofound])
    # the rows behind the addresses are the keys' rows
    sel = np.flatnonzero(fd)[:200]
    rows = read_rows(vp[sel], dim * 4).view(np.float32)
    np.testing.assert_array_equal(rows, values_for(q[sel], dim))


@pytest.mark.parametrize("strategy", ["kLfu", "kCustomized", "kLru", "kEpochLfu"])
def test_find_and_update_matches_oracle(strategy):
    torch, H = _mods()
    st = getattr(H.EvictStrategy, strategy)
    rng = np.random.default_rng(2)
    g, o = make(st, 1 << 13)
    if strategy == "kEpochLfu":
        g.set_global_epoch(3)
        o.set_global_epoch(3)
    uses = strategy != "kLru"
    ks = uniform_keys(rng, 3000)
    insert_both(g, o, ks, 8,
                rng.integers(1, 1 << 30, size=ks.size, dtype=np.uint64) if uses else None,
                clock=40)
    q = np.concatenate([ks[:1500], uniform_keys(rng, 500, exclude=ks), RESERVED])
    inp = rng.integers(1, 1 << 30, size=q.size, dtype=np.uint64) if uses else None
    n = q.size
    vp = torch.zeros(n, dtype=torch.int64, device="cuda")
    fd = torch.zeros(n, dtype=torch.uint8, device="cuda")
    d_sc = to_dev(inp) if uses else None
    g.set_lru_clock(900)
    g.find_and_update(n, to_dev(q), vp, fd, d_sc)
    torch.cuda.synchronize()
    oslots, ofound, oout = o.find_and_update(q, inp, clock=900)
    np.testing.assert_array_equal(to_np(fd, np.uint8).astype(bool), ofound)
    np.testing.assert_array_equal(to_np(vp, np.uint64), expected_ptrs(g, oslots)[1])
    if uses:
        np.testing.assert_array_equal(to_np(d_sc, np.uint64), oout)
    assert_same_layout(g, o, ks)
    with pytest.raises(RuntimeError):
        g.find_and_update(n, to_dev(q), vp, fd, d_sc, unique_key=False)


def _foi_ptr(g, q, scores, unique, keep):
    torch, _ = _mods()
    n = q.size
    vp = torch.zeros(n, dtype=torch.int64, device="cuda")
    fd = torch.zeros(n, dtype=torch.uint8, device="cuda")
    kp = torch.zeros(n, dtype=torch.int64, device="cuda") if keep else None
    g.find_or_insert_ptr(n, to_dev(q), vp, fd,
                         None if scores is None else to_dev(scores), 0, unique,
                         False, kp)
    torch.cuda.synchronize()
    return (to_np(vp, np.uint64), to_np(fd, np.uint8).astype(bool),
            None if kp is None else to_np(kp, np.uint64))


@pytest.mark.parametrize("strategy,unique,keep", [
    ("kCustomized", True, False), ("kCustomized", True, True),
    ("kCustomized", False, False), ("kLfu", True, False), ("kLfu", False, False),
    ("kLru", True, True), ("kLru", False, False), ("kEpochLfu", True, False)])
def test_find_or_insert_ptr_matches_oracle(strategy, unique, keep):
    torch, H = _mods()
    st = getattr(H.EvictStrategy, strategy)
    rng = np.random.default_rng(3)
    dim = 8
    g, o = make(st, 4096, dim=dim)  # 32 buckets: the batches below evict
    if strategy == "kEpochLfu":
        g.set_global_epoch(5)
        o.set_global_epoch(5)
    uses = strategy != "kLru"
    every = []
    for r in range(3):
        ks = uniform_keys(rng, 3000)
        if r:
            ks[:800] = every[-1][:800]  # present keys
        if not unique:
            ks[1000:1400] = ks[:400]  # repeats within the batch
        q = np.concatenate([ks, RESERVED])
        sc = rng.integers(1, 1 << 30, size=q.size, dtype=np.uint64) if uses else None
        clk = 1000 + r
        g.set_lru_clock(clk)
        vp, fd, kp = _foi_ptr(g, q, sc, unique, keep)
        oslots, ofound = o.find_or_insert_ptr(q, sc, unique_key=unique,
                                              keep_locked=keep, clock=clk)
        np.testing.assert_array_equal(fd, ofound)
        ek, ev = expected_ptrs(g, oslots)
        np.testing.assert_array_equal(vp, ev)
        if keep:
            np.testing.assert_array_equal(kp, ek)
            # locked keys are not found; unlocking restores them
            _, f_locked, _, _, of_locked, _ = find_ptr_both(g, o, q)
            np.testing.assert_array_equal(f_locked, of_locked)
            assert not f_locked[oslots != NO].any()
            torch_ok = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
            g.unlock_keys(q.size, to_dev(kp), to_dev(q), torch_ok)
            torch.cuda.synchronize()
            ook = o.unlock_keys(oslots, q)
            np.testing.assert_array_equal(to_np(torch_ok, np.uint8).astype(bool), ook)
            assert ook[oslots != NO].all()
        every.append(ks)
        assert_same_layout(g, o, np.unique(np.concatenate(every)))


@pytest.mark.parametrize("strategy,unique,keep,dups", [
    ("kCustomized", True, False, False), ("kCustomized", True, True, False),
    ("kCustomized", False, False, True), ("kLfu", True, False, False),
    ("kLfu", False, False, True), ("kLru", True, True, False), ("kEpochLfu", False, False, True),
    ("kCustomized", True, False, True), ("kLfu", True, True, True)])
def test_find_or_insert_ptr_single_run(strategy, unique, keep, dups):
    """The pointer find_or_insert on a 512-bucket table with batches under
    one LDS load per partition (the key-parallel single-run kernel): present
    and new keys, repeats (also under unique_key, where a repeat must not
    match the slot its earlier occurrence holds LOCKED), and a table filled
    past full so that buckets go to the eviction kernel."""
    torch, H = _mods()
    st = getattr(H.EvictStrategy, strategy)
    rng = np.random.default_rng(11)
    dim = 8
    cap = 1 << 16
    g, o = make(st, cap, dim=dim)
    if strategy == "kEpochLfu":
        g.set_global_epoch(5)
        o.set_global_epoch(5)
    uses = strategy != "kLru"
    base = uniform_keys(rng, 60000)
    insert_both(g, o, base, dim, rng.integers(1, 1 << 30, size=base.size, dtype=np.uint64)
                if uses else None)
    every = [base]
    for r in range(4):
        ks = np.concatenate([rng.choice(base, 400, replace=False), uniform_keys(rng, 800)])
        if dups:
            ks[900:1000] = ks[:100]  # repeats within the batch
        ks = ks[rng.permutation(ks.size)]
        sc = rng.integers(1, 1 << 30, size=ks.size, dtype=np.uint64) if uses else None
        clk = 2000 + r
        g.set_lru_clock(clk)
        vp, fd, kp = _foi_ptr(g, ks, sc, unique, keep)
        oslots, ofound = o.find_or_insert_ptr(ks, sc, unique_key=unique,
                                              keep_locked=keep, clock=clk)
        np.testing.assert_array_equal(fd, ofound)
        ek, ev = expected_ptrs(g, oslots)
        np.testing.assert_array_equal(vp, ev)
        if keep:
            np.testing.assert_array_equal(kp, ek)
            torch_ok = torch.zeros(ks.size, dtype=torch.uint8, device="cuda")
            g.unlock_keys(ks.size, to_dev(kp), to_dev(ks), torch_ok)
            torch.cuda.synchronize()
            ook = o.unlock_keys(oslots, ks)
            np.testing.assert_array_equal(to_np(torch_ok, np.uint8).astype(bool), ook)
        every.append(ks)
        assert_same_layout(g, o, np.unique(np.concatenate(every)))


def test_rows_written_through_pointers():
    # The reference's find_or_insert_safe_ptr pattern
    # (tests/community/find_or_insert_ptr_lock_test.cpp:152-169): rows of
    # found keys are read through the addresses, rows of new keys written.
    torch, H = _mods()
    rng = np.random.default_rng(4)
    dim = 16
    g, o = make(H.EvictStrategy.kCustomized, 1 << 14, dim=dim)
    old = uniform_keys(rng, 2000)
    insert_both(g, o, old, dim, np.full(old.size, 10, np.uint64))
    q = np.concatenate([old[:500], uniform_keys(rng, 500, exclude=old)])
    vp, fd, kp = _foi_ptr(g, q, np.full(q.size, 20, np.uint64), True, True)
    assert fd[:500].all() and not fd[500:].any()
    got = read_rows(vp[:500], dim * 4).view(np.float32)
    np.testing.assert_array_equal(got, values_for(q[:500], dim))
    write_rows(vp[500:], values_for(q[500:], dim))
    ok = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
    g.unlock_keys(q.size, to_dev(kp), to_dev(q), ok)
    vals = torch.zeros((q.size, dim), dtype=torch.float32, device="cuda")
    founds = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
    g.find(q.size, to_dev(q), vals, founds)
    torch.cuda.synchronize()
    assert to_np(ok, np.uint8).all()
    assert to_np(founds, np.uint8).all()
    np.testing.assert_array_equal(vals.cpu().numpy(), values_for(q, dim))


def test_reference_customized_advanced_kat_on_gpu():
    # tests/community/find_or_insert_ptr_lock_test.cpp:1234-1365 through
    # the library: refused low-score keys, refreshed scores of present keys.
    torch, H = _mods()
    rng = np.random.default_rng(21)
    g, o = make(H.EvictStrategy.kCustomized, 1024, dim=8)
    base = keys_in_bucket(rng, 128, 1024, 0, lo=0, hi=0x3FFFFFFFFFFFFFFF)
    insert_both(g, o, base, 8, np.arange(1000, 1128, dtype=np.uint64))
    test = keys_in_bucket(rng, 8, 1024, 0, lo=0x3FFFFFFFFFFFFFFF,
                          hi=0xFFFFFFFFFFFFFFFD)
    test[4:8] = base[72:76]
    sc = np.array([20, 78, 97, 98, 99, 1010, 1020, 1035], np.uint64)
    vp, fd, kp = _foi_ptr(g, test, sc, True, True)
    assert list(fd) == [False] * 4 + [True] * 4
    assert np.all(vp[:4] == 0) and np.all(kp[:4] == 0) and np.all(vp[4:] != 0)
    ok = torch.zeros(8, dtype=torch.uint8, device="cuda")
    g.unlock_keys(8, to_dev(kp), to_dev(test), ok)
    torch.cuda.synchronize()
    assert list(to_np(ok, np.uint8)) == [0] * 4 + [1] * 4
    o.find_or_insert_ptr(test, sc, keep_locked=False)
    assert_same_layout(g, o, np.concatenate([base, test]))
    assert g.size() == 128


def test_lock_unlock_matches_oracle():
    torch, H = _mods()
    rng = np.random.default_rng(6)
    g, o = make(H.EvictStrategy.kLfu, 1 << 12, dim=8)
    ks = uniform_keys(rng, 2000)
    insert_both(g, o, ks, 8, rng.integers(1, 1 << 30, size=ks.size, dtype=np.uint64))
    q = np.concatenate([ks[:700], uniform_keys(rng, 300, exclude=ks), RESERVED])
    inc = rng.integers(1, 100, size=q.size, dtype=np.uint64)
    n = q.size
    kp = torch.zeros(n, dtype=torch.int64, device="cuda")
    ok = torch.zeros(n, dtype=torch.uint8, device="cuda")
    g.lock_keys(n, to_dev(q), kp, ok, 0, to_dev(inc))
    torch.cuda.synchronize()
    oslots, ook = o.lock_keys(q, inc)
    np.testing.assert_array_equal(to_np(ok, np.uint8).astype(bool), ook)
    kp_np = to_np(kp, np.uint64)
    np.testing.assert_array_equal(kp_np, expected_ptrs(g, oslots)[0])
    # locked keys are invisible to find; a full bucket of locked keys
    # refuses an insert instead of evicting one of them
    _, f, _, _, of, _ = find_ptr_both(g, o, q)
    np.testing.assert_array_equal(f, of)
    # unlock: the real addresses, plus addresses the kernel must reject
    # without writing (null, misaligned inside the key records, foreign)
    other = torch.zeros(4, dtype=torch.int64, device="cuda")
    bad = np.array([0, int(kp_np[0]) + 8, other.data_ptr(),
                    int(kp_np[0]) + 16 * (1 << 30)], np.uint64)
    all_kp = np.concatenate([kp_np, bad])
    all_q = np.concatenate([q, np.arange(4, dtype=np.uint64)])
    ok2 = torch.zeros(all_q.size, dtype=torch.uint8, device="cuda")
    g.unlock_keys(all_q.size, to_dev(all_kp), to_dev(all_q), ok2)
    torch.cuda.synchronize()
    got = to_np(ok2, np.uint8).astype(bool)
    np.testing.assert_array_equal(got[:n], ook)
    assert not got[n:].any()
    assert np.all(other.cpu().numpy() == 0)
    o.unlock_keys(oslots, q)
    assert_same_layout(g, o, ks)


def test_locked_bucket_refuses_inserts():
    torch, H = _mods()
    rng = np.random.default_rng(12)
    g, o = make(H.EvictStrategy.kCustomized, 1024, dim=8)
    base = keys_in_bucket(rng, 128, 1024, 0, lo=0, hi=0x3FFFFFFFFFFFFFFF)
    insert_both(g, o, base, 8, np.arange(1000, 1128, dtype=np.uint64))
    kp = torch.zeros(128, dtype=torch.int64, device="cuda")
    hi = np.full(128, 5000, np.uint64)
    g.lock_keys(128, to_dev(base), kp, None, 0, to_dev(hi))
    oslots, _ = o.lock_keys(base, hi)
    new = keys_in_bucket(rng, 3, 1024, 0, lo=0x4000000000000000,
                         hi=0x7FFFFFFFFFFFFFFF)
    insert_both(g, o, new, 8, np.full(3, 1 << 60, np.uint64))
    _, f, _, _, of, _ = find_ptr_both(g, o, new)
    assert not f.any() and not of.any()
    g.unlock_keys(128, kp, to_dev(base))
    o.unlock_keys(oslots, base)
    insert_both(g, o, new, 8, np.full(3, 1 << 60, np.uint64))
    assert_same_layout(g, o, np.concatenate([base, new]))


def test_find_or_insert_ptr_grows_table():
    torch, H = _mods()
    rng = np.random.default_rng(7)
    g, o = make(H.EvictStrategy.kCustomized, 1024, max_cap=1 << 14, dim=8)
    every = []
    for r in range(4):
        ks = uniform_keys(rng, 1500)
        sc = rng.integers(1, 1 << 30, size=ks.size, dtype=np.uint64)
        vp, fd, _ = _foi_ptr(g, ks, sc, True, False)
        oslots, ofound = o.find_or_insert_ptr(ks, sc)
        assert g.capacity() == o.capacity()
        np.testing.assert_array_equal(fd, ofound)
        np.testing.assert_array_equal(vp, expected_ptrs(g, oslots)[1])
        every.append(ks)
    assert g.capacity() > 1024
    assert_same_layout(g, o, np.concatenate(every))


def test_pointer_api_argument_errors():
    torch, H = _mods()
    g, _ = make(H.EvictStrategy.kCustomized, 1024)
    q = to_dev(np.arange(4, dtype=np.uint64))
    vp = torch.zeros(4, dtype=torch.int64, device="cuda")
    fd = torch.zeros(4, dtype=torch.uint8, device="cuda")
    kp = torch.zeros(4, dtype=torch.int64, device="cuda")
    sc = to_dev(np.ones(4, np.uint64))
    with pytest.raises(H.UnsupportedError):
        g.find_or_insert_ptr(4, q, vp, fd, sc, 0, False, False, kp)
    with pytest.raises(H.HkvException):
        g.find_or_insert_ptr(4, q, vp, fd, None)  # Customized needs scores
    with pytest.raises(H.HkvException):
        g.lock_keys(4, q, kp)  # Customized needs scores
    g.find_or_insert_ptr(0, q, vp, fd, sc)  # n == 0 is a no-op
