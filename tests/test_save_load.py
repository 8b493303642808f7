"""save / load (include/hkv_hashtable.h:3021-3195) and the LocalKVFile format
(include/types.h:350-464: three raw files of keys, rows and scores).

save writes the live records in slot order, in chunks of
max_workspace_size / (key + score + row) slots; load reads chunks of that
many records and applies each as insert_or_assign(unique_key=true,
ignore_evict_strategy=true) with the global epoch set to IGNORED.  The GPU
tests compare the saved files with the oracle's slot-order export and the
loaded table with the oracle driven through the same chunked calls.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import uniform_keys


def rand_vals(rng, n, dim):
    return rng.uniform(-1, 1, (n, dim)).astype(np.float32)


def chunk_records(max_ws, dim, vsize=4):
    return max_ws // (8 + 8 + dim * vsize)


def oracle_load(o, keys, values, scores, max_ws):
    """The reference's load loop on the oracle."""
    n = chunk_records(max_ws, o.dim)
    for i in range(0, keys.size, n):
        o.set_global_epoch(O.IGNORED_GLOBAL_EPOCH)
        o.insert_or_assign(keys[i:i + n], values[i:i + n], scores[i:i + n], True, True, 0)


def paths(tmp_path, tag):
    return [str(tmp_path / f"{tag}.{x}") for x in ("keys", "values", "scores")]


def read_files(ps, dim):
    k = np.fromfile(ps[0], np.uint64)
    v = np.fromfile(ps[1], np.float32).reshape(-1, dim)
    s = np.fromfile(ps[2], np.uint64)
    return k, v, s


def test_local_kv_file_format(tmp_path):
    """The file helpers (no GPU): raw arrays, appended chunk by chunk; a
    read returns 0 once the three files run short together."""
    import ctypes
    import hkv_amd
    L = hkv_amd._LIB
    ps = paths(tmp_path, "fmt")
    rng = np.random.default_rng(1)
    k = rng.integers(0, 2**63, 100, dtype=np.uint64)
    v = rng.uniform(-1, 1, (100, 3)).astype(np.float32)
    s = rng.integers(0, 2**63, 100, dtype=np.uint64)
    f = L.hkv_local_kv_file_open(*(p.encode() for p in ps), b"wb")
    assert f
    for a, b in ((0, 60), (60, 100)):
        assert L.hkv_local_kv_file_write(f, b - a, 12, k[a:].ctypes.data, v[a:].ctypes.data,
                                         s[a:].ctypes.data) == b - a
    L.hkv_local_kv_file_close(f)
    gk, gv, gs = read_files(ps, 3)
    np.testing.assert_array_equal(gk, k)
    np.testing.assert_array_equal(gv, v)
    np.testing.assert_array_equal(gs, s)
    f = L.hkv_local_kv_file_open(*(p.encode() for p in ps), b"rb")
    rk = np.zeros(70, np.uint64)
    rv = np.zeros((70, 3), np.float32)
    rs = np.zeros(70, np.uint64)
    assert L.hkv_local_kv_file_read(f, 70, 12, rk.ctypes.data, rv.ctypes.data,
                                    rs.ctypes.data) == 70
    assert L.hkv_local_kv_file_read(f, 70, 12, rk.ctypes.data, rv.ctypes.data,
                                    rs.ctypes.data) == 30
    assert L.hkv_local_kv_file_read(f, 70, 12, rk.ctypes.data, rv.ctypes.data,
                                    rs.ctypes.data) == 0
    np.testing.assert_array_equal(rk[:30], k[70:])
    L.hkv_local_kv_file_close(f)
    assert not L.hkv_local_kv_file_open(b"/nonexistent/dir/k", b"/x", b"/y", b"rb")
    del ctypes


@pytest.mark.gpu
@pytest.mark.parametrize("strategy,max_ws", [(O.CUSTOMIZED, 50_000), (O.LRU, 1 << 20),
                                             (O.LFU, 4096)])
def test_save_then_load(tmp_path, strategy, max_ws):
    import hkv_amd
    from gpu_pair import Pair
    rng = np.random.default_rng(400 + strategy)
    dim = 16
    p = Pair(1 << 13, 1 << 15, dim=dim, strategy=strategy)
    for b in range(4):
        ks = uniform_keys(rng, 2500)
        p.insert_or_assign(ks, rand_vals(rng, ks.size, dim),
                           None if strategy == O.LRU else
                           rng.integers(0, 1 << 40, ks.size, dtype=np.uint64), clock=9 + b)
    ps = paths(tmp_path, "save")
    f = hkv_amd.LocalKVFile()
    assert f.open(*ps, "wb")
    n = p.g.save(f, max_ws)
    f.close()
    ok, ov, os_ = p.o.export_batch(p.o.capacity(), 0)
    assert n == ok.size == p.g.size()
    gk, gv, gs = read_files(ps, dim)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv.view(np.uint32), ov.view(np.uint32))
    np.testing.assert_array_equal(gs, os_)
    # load into a fresh table (growth happens between chunks) and into one
    # that already holds other keys
    for pre in (0, 3000):
        q = Pair(1 << 12, 1 << 15, dim=dim, strategy=O.EPOCH_LFU)
        if pre:
            q.set_global_epoch(2)
            ks = uniform_keys(rng, pre)
            q.insert_or_assign(ks, rand_vals(rng, pre, dim),
                               rng.integers(0, 100, pre, dtype=np.uint64))
            q.insert_or_assign(gk[:500].copy(), rand_vals(rng, 500, dim),
                               rng.integers(0, 100, 500, dtype=np.uint64))
        f = hkv_amd.LocalKVFile()
        assert f.open(*ps, "rb")
        m = q.g.load(f, max_ws)
        f.close()
        assert m == gk.size
        oracle_load(q.o, gk, gv, gs, max_ws)
        q.assert_same_state()


@pytest.mark.gpu
def test_save_load_hybrid_and_python_file(tmp_path):
    """A table with rows in pinned host memory, saved through a Python
    BaseKVFile (records kept in memory) and loaded back."""
    import hkv_amd
    from gpu_pair import Pair
    rng = np.random.default_rng(410)
    dim = 64
    p = Pair(1 << 15, dim=dim, strategy=O.CUSTOMIZED, max_hbm=2 << 20)
    assert not p.g.is_pure_hbm_mode()
    ks = uniform_keys(rng, 12000)
    p.insert_or_assign(ks, rand_vals(rng, ks.size, dim),
                       rng.integers(0, 1 << 40, ks.size, dtype=np.uint64))

    class MemFile(hkv_amd.BaseKVFile):
        def __init__(self):
            self.k, self.v, self.s, self.pos = [], [], [], 0

        def write(self, n, d, keys, values, scores):
            self.k.append(keys.copy())
            self.v.append(values.copy())
            self.s.append(scores.copy())
            return n

        def read(self, n, d, keys, values, scores):
            k = np.concatenate(self.k)
            m = min(n, k.size - self.pos)
            keys[:m] = k[self.pos:self.pos + m]
            values[:m] = np.concatenate(self.v)[self.pos:self.pos + m]
            scores[:m] = np.concatenate(self.s)[self.pos:self.pos + m]
            self.pos += m
            return m
    mf = MemFile()
    assert p.g.save(mf, 100_000) == ks.size
    ok, ov, os_ = p.o.export_batch(p.o.capacity(), 0)
    np.testing.assert_array_equal(np.concatenate(mf.k), ok)
    np.testing.assert_array_equal(np.concatenate(mf.v).view(np.uint32), ov.view(np.uint32))
    np.testing.assert_array_equal(np.concatenate(mf.s), os_)
    q = Pair(1 << 15, dim=dim, strategy=O.LFU, max_hbm=2 << 20)
    assert q.g.load(mf, 100_000) == ks.size
    oracle_load(q.o, ok, ov, os_, 100_000)
    q.assert_same_state()
    with pytest.raises(hkv_amd.HkvException):
        q.g.save(mf, 100)  # below one key + score + row
