"""Runs the same operations on the gfx950 table (through the C ABI) and on
the oracle, and compares results bit-exactly."""
import numpy as np

import oracle as O

TORCH_DT = None


def _torch():
    import torch
    return torch


NP_OF = {"f32": np.float32, "f64": np.float64, "f16": np.float16,
         "bf16": np.uint16, "i8": np.int8, "u8": np.uint8, "i16": np.int16,
         "u16": np.uint16, "i32": np.int32, "u32": np.uint32, "i64": np.int64,
         "u64": np.uint64}


def to_dev(a):
    torch = _torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint64:
        a = a.view(np.int64)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.bool_:
        a = a.astype(np.uint8)
    return torch.from_numpy(a.copy()).cuda()


def to_np(t, dtype):
    return t.cpu().numpy().view(dtype)


class Pair:
    BIG_HBM = 1 << 40

    def __init__(self, init_capacity, max_capacity=None, dim=16,
                 strategy=O.CUSTOMIZED, vt="f32", max_hbm=None,
                 max_load_factor=0.5, oracle_threads=1):
        import hkv_amd
        torch = _torch()
        self.torch = torch
        self.dim, self.vt, self.np_vt = dim, vt, NP_OF[vt]
        if max_capacity is None:
            max_capacity = init_capacity
        self.o = O.Oracle(init_capacity, max_capacity, dim=dim,
                          strategy=strategy, value_type=vt,
                          max_load_factor=max_load_factor,
                          threads=oracle_threads)
        self.g = hkv_amd.HashTable("u64", vt, strategy)
        self.g.init(hkv_amd.HashTableOptions(
            init_capacity=init_capacity, max_capacity=max_capacity,
            max_hbm_for_vectors=self.BIG_HBM if max_hbm is None else max_hbm,
            dim=dim, max_load_factor=max_load_factor))
        self.strategy = strategy

    def set_global_epoch(self, e):
        self.o.set_global_epoch(e)
        self.g.set_global_epoch(e)

    def _vals(self, v, n):
        return np.ascontiguousarray(v, dtype=self.np_vt).reshape(n, self.dim)

    # -- mutating ops ----------------------------------------------------
    def insert_or_assign(self, keys, values, scores=None, unique_key=True,
                         ignore=False, clock=12345):
        n = keys.size
        v = self._vals(values, n)
        self.o.insert_or_assign(keys, v, scores, unique_key, ignore, clock)
        self.g.set_lru_clock(clock)
        self.g.insert_or_assign(n, to_dev(keys), to_dev(v),
                                None if scores is None else to_dev(scores),
                                0, unique_key, ignore)

    def find_or_insert(self, keys, values, scores=None, unique_key=True,
                       clock=12345, ignore=False):
        n = keys.size
        v = self._vals(values, n)
        ov = self.o.find_or_insert(keys, v, scores, unique_key, ignore, clock)
        gv = to_dev(v)
        self.g.set_lru_clock(clock)
        self.g.find_or_insert(n, to_dev(keys), gv,
                              None if scores is None else to_dev(scores), 0,
                              unique_key, ignore)
        return ov, to_np(gv, self.np_vt).reshape(n, self.dim)

    def insert_and_evict(self, keys, values, scores=None, unique_key=True,
                         clock=12345):
        n = keys.size
        v = self._vals(values, n)
        ok, ov, os_ = self.o.insert_and_evict(keys, v, scores, unique_key,
                                              False, clock)
        torch = self.torch
        ek = torch.zeros(n, dtype=torch.int64, device="cuda")
        ev = to_dev(np.zeros((n, self.dim), self.np_vt))
        es = torch.zeros(n, dtype=torch.int64, device="cuda")
        self.g.set_lru_clock(clock)
        c = self.g.insert_and_evict(n, to_dev(keys), to_dev(v),
                                    None if scores is None else to_dev(scores),
                                    ek, ev, es, None, 0, unique_key)
        gk = to_np(ek, np.uint64)[:c]
        gv = to_np(ev, self.np_vt).reshape(n, self.dim)[:c]
        gs = to_np(es, np.uint64)[:c]
        return (ok, ov, os_), (gk, gv, gs)

    def accum_or_assign(self, keys, values, flags, scores=None, clock=12345):
        n = keys.size
        v = self._vals(values, n)
        self.o.accum_or_assign(keys, v, flags, scores, False, clock)
        self.g.set_lru_clock(clock)
        self.g.accum_or_assign(n, to_dev(keys), to_dev(v),
                               to_dev(np.asarray(flags, np.uint8)),
                               None if scores is None else to_dev(scores))

    def assign_scores(self, keys, scores=None, clock=12345):
        self.o.assign_scores(keys, scores, clock)
        self.g.set_lru_clock(clock)
        self.g.assign_scores(keys.size, to_dev(keys),
                             None if scores is None else to_dev(scores))

    def erase(self, keys):
        self.o.erase(keys)
        self.g.erase(keys.size, to_dev(keys))

    def clear(self):
        self.o.clear()
        self.g.clear()

    def reserve(self, c):
        self.o.reserve(c)
        self.g.reserve(c)

    # -- reads -----------------------------------------------------------
    def find(self, keys, fill=0):
        n = keys.size
        init = np.full((n, self.dim), fill, self.np_vt)
        ov, of, os_ = self.o.find(keys, init.copy(), with_scores=True)
        torch = self.torch
        gv = to_dev(init)
        gf = torch.zeros(n, dtype=torch.uint8, device="cuda")
        gs = torch.zeros(n, dtype=torch.int64, device="cuda")
        self.g.find(n, to_dev(keys), gv, gf, gs)
        return ((ov, of, os_),
                (to_np(gv, self.np_vt).reshape(n, self.dim),
                 to_np(gf, np.uint8).astype(bool), to_np(gs, np.uint64)))

    def export(self, n=None, offset=0):
        cap = self.g.capacity()
        if n is None:
            n = cap
        m = max(0, min(n, cap - offset))
        torch = self.torch
        gk = torch.zeros(max(m, 1), dtype=torch.int64, device="cuda")
        gv = to_dev(np.zeros((max(m, 1), self.dim), self.np_vt))
        gs = torch.zeros(max(m, 1), dtype=torch.int64, device="cuda")
        c = self.g.export_batch(n, offset, gk, gv, gs)
        g = (to_np(gk, np.uint64)[:c],
             to_np(gv, self.np_vt).reshape(-1, self.dim)[:c],
             to_np(gs, np.uint64)[:c])
        return self.o.export_batch(n, offset), g

    # -- checks ----------------------------------------------------------
    def assert_same_state(self):
        assert self.g.capacity() == self.o.capacity()
        assert self.g.size() == self.o.size()
        assert self.g.live_count() == self.o.size()
        (ok, ov, os_), (gk, gv, gs) = self.export()
        np.testing.assert_array_equal(gk, ok)
        np.testing.assert_array_equal(gs, os_)
        np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))

    def assert_same_find(self, keys, fill=0):
        (ov, of, os_), (gv, gf, gs) = self.find(keys, fill)
        np.testing.assert_array_equal(gf, of)
        np.testing.assert_array_equal(gv.view(np.uint8), ov.view(np.uint8))
        np.testing.assert_array_equal(gs[of], os_[of])
        return of


def records_equal(o, g):
    """Evicted-record multisets equal: (key, score, row bytes) as one sort
    key, since record order is unspecified and a key can leave two records
    with the same score in one call (evicted, then refused)."""
    ok, ov, os_ = o
    gk, gv, gs = g
    assert gk.size == ok.size
    if ok.size == 0:
        return

    def table(k, v, s):
        return np.concatenate([k.reshape(-1, 1).view(np.uint8), s.reshape(-1, 1).view(np.uint8),
                               np.ascontiguousarray(v).reshape(k.size, -1).view(np.uint8)],
                              axis=1)
    a, b = table(ok, ov, os_), table(gk, gv, gs)
    a = a[np.lexsort(a.T[::-1])] if a.size else a
    b = b[np.lexsort(b.T[::-1])] if b.size else b
    np.testing.assert_array_equal(b, a)


class GpuTable:
    """The gfx950 table (through the C ABI) behind the oracle's numpy-facing
    method names, so that a known-answer test written against the oracle can
    run unchanged against the GPU."""

    def __init__(self, init_capacity, max_capacity=None, dim=16,
                 max_bucket_size=128, strategy=O.LRU, value_type="f32",
                 max_load_factor=0.5, threads=1):
        import hkv_amd
        if max_capacity is None:
            max_capacity = init_capacity
        self.torch = _torch()
        self.dim, self.np_vt = dim, NP_OF[value_type]
        self.g = hkv_amd.HashTable("u64", value_type, strategy)
        self.g.init(hkv_amd.HashTableOptions(
            init_capacity=init_capacity, max_capacity=max_capacity,
            max_hbm_for_vectors=Pair.BIG_HBM, dim=dim,
            max_bucket_size=max_bucket_size, max_load_factor=max_load_factor))

    def _v(self, values, n):
        return np.ascontiguousarray(values, dtype=self.np_vt).reshape(n, self.dim)

    @staticmethod
    def _s(scores):
        return None if scores is None else to_dev(np.asarray(scores, np.uint64))

    def set_global_epoch(self, e):
        self.g.set_global_epoch(e)

    def insert_or_assign(self, keys, values, scores=None, unique_key=True,
                         ignore_evict_strategy=False, clock=0):
        keys = np.asarray(keys, np.uint64)
        self.g.set_lru_clock(clock)
        self.g.insert_or_assign(keys.size, to_dev(keys), to_dev(self._v(values, keys.size)),
                                self._s(scores), 0, unique_key, ignore_evict_strategy)

    def find_or_insert(self, keys, values, scores=None, unique_key=True,
                       ignore_evict_strategy=False, clock=0):
        keys = np.asarray(keys, np.uint64)
        v = to_dev(self._v(values, keys.size))
        self.g.set_lru_clock(clock)
        self.g.find_or_insert(keys.size, to_dev(keys), v, self._s(scores), 0,
                              unique_key, ignore_evict_strategy)
        return to_np(v, self.np_vt).reshape(keys.size, self.dim)

    def accum_or_assign(self, keys, values, accum, scores=None,
                        ignore_evict_strategy=False, clock=0):
        keys = np.asarray(keys, np.uint64)
        self.g.set_lru_clock(clock)
        self.g.accum_or_assign(keys.size, to_dev(keys), to_dev(self._v(values, keys.size)),
                               to_dev(np.asarray(accum, np.uint8)), self._s(scores), 0,
                               ignore_evict_strategy)

    def assign_scores(self, keys, scores=None, clock=0):
        keys = np.asarray(keys, np.uint64)
        self.g.set_lru_clock(clock)
        self.g.assign_scores(keys.size, to_dev(keys), self._s(scores))

    def find(self, keys, values=None, with_scores=False):
        torch = self.torch
        keys = np.asarray(keys, np.uint64)
        n = keys.size
        if values is None:
            values = np.zeros((n, self.dim), self.np_vt)
        v = to_dev(values)
        f = torch.zeros(n, dtype=torch.uint8, device="cuda")
        s = torch.zeros(n, dtype=torch.int64, device="cuda") if with_scores else None
        self.g.find(n, to_dev(keys), v, f, s)
        return (to_np(v, self.np_vt).reshape(n, self.dim), to_np(f, np.uint8).astype(bool),
                None if s is None else to_np(s, np.uint64))

    def export_batch(self, n, offset=0):
        torch = self.torch
        m = max(1, min(n, self.g.capacity() - offset))
        k = torch.zeros(m, dtype=torch.int64, device="cuda")
        v = to_dev(np.zeros((m, self.dim), self.np_vt))
        s = torch.zeros(m, dtype=torch.int64, device="cuda")
        c = self.g.export_batch(n, offset, k, v, s)
        return (to_np(k, np.uint64)[:c], to_np(v, self.np_vt).reshape(m, self.dim)[:c],
                to_np(s, np.uint64)[:c])

    def size(self):
        return self.g.size()

    def capacity(self):
        return self.g.capacity()
