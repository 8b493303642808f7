"""ctypes wrapper around liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is the host C++ restatement of the HierarchicalKV-ascend table
(oracle/hkv_oracle.cpp).  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module; it is the checker,
never the thing measured or shipped.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

LRU, LFU, EPOCH_LRU, EPOCH_LFU, CUSTOMIZED = 0, 1, 2, 3, 4
IGNORED_GLOBAL_EPOCH = 0xFFFFFFFFFFFFFFFF

VT = {"f32": 0, "f64": 1, "f16": 2, "bf16": 3, "i8": 4, "u8": 5, "i16": 6,
      "u16": 7, "i32": 8, "u32": 9, "i64": 10, "u64": 11}
NP = {"f32": np.float32, "f64": np.float64, "f16": np.float16,
      "bf16": np.uint16, "i8": np.int8, "u8": np.uint8, "i16": np.int16,
      "u16": np.uint16, "i32": np.int32, "u32": np.uint32, "i64": np.int64,
      "u64": np.uint64}

u64p = ctypes.POINTER(ctypes.c_uint64)
vp = ctypes.c_void_p


def build():
    subprocess.check_call(["make", "-s", "-C", _HERE, "liboracle.so"])


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.hkvo_create.restype = vp
        L.hkvo_create.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                  ctypes.c_uint64, ctypes.c_uint64,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                  ctypes.POINTER(ctypes.c_int)]
        L.hkvo_destroy.argtypes = [vp]
        L.hkvo_set_threads.argtypes = [vp, ctypes.c_int]
        L.hkvo_set_global_epoch.argtypes = [vp, ctypes.c_uint64]
        L.hkvo_insert_or_assign.argtypes = [vp, ctypes.c_uint64, vp, vp, vp,
                                            ctypes.c_int, ctypes.c_int,
                                            ctypes.c_uint64]
        L.hkvo_find.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp]
        L.hkvo_find_missed.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp,
                                       vp, vp]
        L.hkvo_find_or_insert.argtypes = [vp, ctypes.c_uint64, vp, vp, vp,
                                          ctypes.c_int, ctypes.c_int,
                                          ctypes.c_uint64]
        L.hkvo_insert_and_evict.argtypes = [vp, ctypes.c_uint64, vp, vp, vp,
                                            vp, vp, vp, vp, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_uint64]
        L.hkvo_accum_or_assign.argtypes = [vp, ctypes.c_uint64, vp, vp, vp,
                                           vp, ctypes.c_int, ctypes.c_uint64]
        L.hkvo_assign_scores.argtypes = [vp, ctypes.c_uint64, vp, vp,
                                         ctypes.c_uint64]
        L.hkvo_erase.argtypes = [vp, ctypes.c_uint64, vp]
        L.hkvo_clear.argtypes = [vp]
        L.hkvo_export_batch.restype = ctypes.c_uint64
        L.hkvo_export_batch.argtypes = [vp, ctypes.c_uint64, ctypes.c_uint64,
                                        vp, vp, vp]
        L.hkvo_reserve.argtypes = [vp, ctypes.c_uint64]
        for f in ("hkvo_size", "hkvo_capacity", "hkvo_bucket_count"):
            getattr(L, f).restype = ctypes.c_uint64
            getattr(L, f).argtypes = [vp]
        L.hkvo_raw.argtypes = [vp] + [ctypes.POINTER(vp)] * 5
        L.hkvo_murmur3.restype = ctypes.c_uint64
        L.hkvo_murmur3.argtypes = [ctypes.c_uint64]
        L.hkvo_global_idx.restype = ctypes.c_uint64
        L.hkvo_global_idx.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.hkvo_empty_digest.restype = ctypes.c_uint8
        L.hkvo_reclaim_digest.restype = ctypes.c_uint8
        L.hkvo_score_desired.restype = ctypes.c_uint64
        L.hkvo_score_desired.argtypes = [ctypes.c_int, ctypes.c_int,
                                         ctypes.c_uint64, ctypes.c_uint64,
                                         ctypes.c_uint64]
        for f in ("hkvo_score_new", "hkvo_score_hit"):
            getattr(L, f).restype = ctypes.c_uint64
            getattr(L, f).argtypes = [ctypes.c_int, ctypes.c_int,
                                      ctypes.c_uint64, ctypes.c_uint64,
                                      ctypes.c_uint64]
        L.hkvo_score_without_missed.restype = ctypes.c_uint64
        L.hkvo_score_without_missed.argtypes = [ctypes.c_int, ctypes.c_int,
                                                ctypes.c_uint64,
                                                ctypes.c_uint64,
                                                ctypes.c_uint64,
                                                ctypes.c_uint64]
        L.hkvo_erase_if.argtypes = [vp, ctypes.c_int, ctypes.c_uint64,
                                    ctypes.c_uint64, ctypes.c_int, vp]
        L.hkvo_size_if.argtypes = [vp, ctypes.c_int, ctypes.c_uint64,
                                   ctypes.c_uint64, ctypes.c_int, vp]
        L.hkvo_export_batch_if.restype = ctypes.c_uint64
        L.hkvo_export_batch_if.argtypes = [vp, ctypes.c_int, ctypes.c_uint64,
                                           ctypes.c_uint64, ctypes.c_int,
                                           ctypes.c_uint64, ctypes.c_uint64,
                                           vp, vp, vp]
        L.hkvo_set_max_capacity.argtypes = [vp, ctypes.c_uint64]
        L.hkvo_contains.argtypes = [vp, ctypes.c_uint64, vp, vp]
        L.hkvo_assign.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, ctypes.c_int,
                                  ctypes.c_uint64]
        L.hkvo_find_ptr.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp]
        L.hkvo_find_and_update.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp,
                                           ctypes.c_int, ctypes.c_uint64]
        L.hkvo_find_or_insert_ptr.argtypes = [vp, ctypes.c_uint64, vp, vp, vp,
                                              vp, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_uint64]
        L.hkvo_lock_keys.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp,
                                     ctypes.c_uint64]
        L.hkvo_unlock_keys.argtypes = [vp, ctypes.c_uint64, vp, vp, vp]
        _LIB = L
    return _LIB


NO_SLOT = 0xFFFFFFFFFFFFFFFF


def _p(a):
    return None if a is None else a.ctypes.data_as(vp)


class OracleError(RuntimeError):
    def __init__(self, code):
        super().__init__("oracle status %d" % code)
        self.code = code


def _chk(rc):
    if rc:
        raise OracleError(rc)


class Oracle:
    """Host reference table with the same method names as the product."""

    def __init__(self, init_capacity, max_capacity=None, dim=16,
                 max_bucket_size=128, strategy=LRU, value_type="f32",
                 max_load_factor=0.5, threads=1):
        L = lib()
        st = ctypes.c_int(0)
        if max_capacity is None:
            max_capacity = init_capacity
        self.dim = dim
        self.vt = value_type
        self.np_vt = NP[value_type]
        self.h = L.hkvo_create(init_capacity, max_capacity, max_bucket_size,
                               dim, VT[value_type], strategy,
                               max_load_factor, ctypes.byref(st))
        _chk(st.value)
        if threads != 1:
            L.hkvo_set_threads(self.h, threads)

    def __del__(self):
        if getattr(self, "h", None):
            lib().hkvo_destroy(self.h)
            self.h = None

    def set_threads(self, t):
        lib().hkvo_set_threads(self.h, t)

    def set_global_epoch(self, e):
        lib().hkvo_set_global_epoch(self.h, e)

    def _vals(self, values, n):
        v = np.ascontiguousarray(values, dtype=self.np_vt).reshape(n, self.dim)
        return v

    def insert_or_assign(self, keys, values, scores=None, unique_key=True,
                         ignore_evict_strategy=False, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        v = self._vals(values, n)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_insert_or_assign(self.h, n, _p(keys), _p(v), _p(s),
                                         int(unique_key),
                                         int(ignore_evict_strategy), clock))

    def find(self, keys, values=None, with_scores=False):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        if values is None:
            values = np.zeros((n, self.dim), self.np_vt)
        founds = np.zeros(n, np.uint8)
        scores = np.zeros(n, np.uint64) if with_scores else None
        _chk(lib().hkvo_find(self.h, n, _p(keys), _p(values), _p(founds),
                             _p(scores)))
        return values, founds.astype(bool), scores

    def find_missed(self, keys, values=None, with_scores=False):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        if values is None:
            values = np.zeros((n, self.dim), self.np_vt)
        mk = np.zeros(n, np.uint64)
        mi = np.zeros(n, np.int32)
        ms = np.zeros(1, np.int32)
        scores = np.zeros(n, np.uint64) if with_scores else None
        _chk(lib().hkvo_find_missed(self.h, n, _p(keys), _p(values), _p(mk),
                                    _p(mi), _p(ms), _p(scores)))
        m = int(ms[0])
        return values, mk[:m], mi[:m], scores

    def find_or_insert(self, keys, values, scores=None, unique_key=True,
                       ignore_evict_strategy=False, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        v = np.array(values, dtype=self.np_vt).reshape(n, self.dim)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_find_or_insert(self.h, n, _p(keys), _p(v), _p(s),
                                       int(unique_key),
                                       int(ignore_evict_strategy), clock))
        return v

    def insert_and_evict(self, keys, values, scores=None, unique_key=True,
                         ignore_evict_strategy=False, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        v = self._vals(values, n)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        ek = np.zeros(n, np.uint64)
        ev = np.zeros((n, self.dim), self.np_vt)
        es = np.zeros(n, np.uint64)
        cnt = np.zeros(1, np.uint64)
        _chk(lib().hkvo_insert_and_evict(self.h, n, _p(keys), _p(v), _p(s),
                                         _p(ek), _p(ev), _p(es), _p(cnt),
                                         int(unique_key),
                                         int(ignore_evict_strategy), clock))
        c = int(cnt[0])
        return ek[:c], ev[:c], es[:c]

    def accum_or_assign(self, keys, values, accum, scores=None,
                        ignore_evict_strategy=False, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        v = self._vals(values, n)
        a = np.ascontiguousarray(accum, dtype=np.uint8)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_accum_or_assign(self.h, n, _p(keys), _p(v), _p(a),
                                        _p(s), int(ignore_evict_strategy),
                                        clock))

    def assign_scores(self, keys, scores=None, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_assign_scores(self.h, keys.size, _p(keys), _p(s),
                                      clock))

    # --- predicates: built-in kinds 0..4 (see include/hkv_amd.h) -----------
    def erase_if(self, pred, pattern, threshold, key_signed=False):
        c = np.zeros(1, np.uint64)
        _chk(lib().hkvo_erase_if(self.h, pred, pattern, threshold,
                                 int(key_signed), _p(c)))
        return int(c[0])

    def size_if(self, pred, pattern, threshold, key_signed=False):
        c = np.zeros(1, np.uint64)
        _chk(lib().hkvo_size_if(self.h, pred, pattern, threshold,
                                int(key_signed), _p(c)))
        return int(c[0])

    def export_batch_if(self, pred, pattern, threshold, n, offset=0,
                        key_signed=False):
        cap = self.capacity()
        m = max(0, min(n, cap - offset)) if offset < cap else 0
        k = np.zeros(m, np.uint64)
        v = np.zeros((m, self.dim), self.np_vt)
        s = np.zeros(m, np.uint64)
        c = lib().hkvo_export_batch_if(self.h, pred, pattern, threshold,
                                       int(key_signed), n, offset, _p(k), _p(v),
                                       _p(s))
        return k[:c], v[:c], s[:c]

    def set_max_capacity(self, new_max):
        _chk(lib().hkvo_set_max_capacity(self.h, new_max))

    def contains(self, keys):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        f = np.zeros(keys.size, np.uint8)
        _chk(lib().hkvo_contains(self.h, keys.size, _p(keys), _p(f)))
        return f.astype(bool)

    def assign(self, keys, values, scores=None, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        v = self._vals(values, keys.size)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_assign(self.h, keys.size, _p(keys), _p(v), _p(s), 1, clock))

    def assign_values(self, keys, values):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        v = self._vals(values, keys.size)
        _chk(lib().hkvo_assign(self.h, keys.size, _p(keys), _p(v), None, 0, 0))

    # --- pointer APIs: global slot indices (NO_SLOT for none) ----------------
    def find_ptr(self, keys, with_scores=False):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        slots = np.zeros(n, np.uint64)
        founds = np.zeros(n, np.uint8)
        scores = np.zeros(n, np.uint64) if with_scores else None
        _chk(lib().hkvo_find_ptr(self.h, n, _p(keys), _p(slots), _p(founds),
                                 _p(scores)))
        return slots, founds.astype(bool), scores

    def find_and_update(self, keys, scores=None, unique_key=True, clock=0):
        """Returns (slots, founds, scores after the call)."""
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        slots = np.zeros(n, np.uint64)
        founds = np.zeros(n, np.uint8)
        s = None if scores is None else np.array(scores, np.uint64)
        _chk(lib().hkvo_find_and_update(self.h, n, _p(keys), _p(slots),
                                        _p(founds), _p(s), int(unique_key),
                                        clock))
        return slots, founds.astype(bool), s

    def find_or_insert_ptr(self, keys, scores=None, unique_key=True,
                           ignore_evict_strategy=False, keep_locked=False,
                           clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        slots = np.zeros(n, np.uint64)
        founds = np.zeros(n, np.uint8)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_find_or_insert_ptr(self.h, n, _p(keys), _p(slots),
                                           _p(founds), _p(s), int(unique_key),
                                           int(ignore_evict_strategy),
                                           int(keep_locked), clock))
        return slots, founds.astype(bool)

    def lock_keys(self, keys, scores=None, clock=0):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        n = keys.size
        slots = np.zeros(n, np.uint64)
        ok = np.zeros(n, np.uint8)
        s = None if scores is None else np.ascontiguousarray(scores, np.uint64)
        _chk(lib().hkvo_lock_keys(self.h, n, _p(keys), _p(slots), _p(ok), _p(s),
                                  clock))
        return slots, ok.astype(bool)

    def unlock_keys(self, slots, keys):
        slots = np.ascontiguousarray(slots, dtype=np.uint64)
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        ok = np.zeros(keys.size, np.uint8)
        _chk(lib().hkvo_unlock_keys(self.h, keys.size, _p(slots), _p(keys),
                                    _p(ok)))
        return ok.astype(bool)

    def erase(self, keys):
        keys = np.ascontiguousarray(keys, dtype=np.uint64)
        _chk(lib().hkvo_erase(self.h, keys.size, _p(keys)))

    def clear(self):
        lib().hkvo_clear(self.h)

    def export_batch(self, n, offset=0):
        cap = self.capacity()
        m = max(0, min(n, cap - offset)) if offset < cap else 0
        k = np.zeros(m, np.uint64)
        v = np.zeros((m, self.dim), self.np_vt)
        s = np.zeros(m, np.uint64)
        c = lib().hkvo_export_batch(self.h, n, offset, _p(k), _p(v), _p(s))
        return k[:c], v[:c], s[:c]

    def reserve(self, new_capacity):
        _chk(lib().hkvo_reserve(self.h, new_capacity))

    def size(self):
        return int(lib().hkvo_size(self.h))

    def capacity(self):
        return int(lib().hkvo_capacity(self.h))

    def bucket_count(self):
        return int(lib().hkvo_bucket_count(self.h))

    def load_factor(self):
        return self.size() / self.capacity()

    def raw(self, bucket_size=128):
        """Copies of (digests, keys, scores, bucket_sizes, values)."""
        ptrs = [vp() for _ in range(5)]
        lib().hkvo_raw(self.h, *[ctypes.byref(p) for p in ptrs])
        cap, nb = self.capacity(), self.bucket_count()

        def arr(p, dt, cnt):
            buf = (ctypes.c_char * (np.dtype(dt).itemsize * cnt)).from_address(
                p.value)
            return np.frombuffer(buf, dtype=dt, count=cnt).copy()
        d = arr(ptrs[0], np.uint8, cap)
        k = arr(ptrs[1], np.uint64, cap)
        s = arr(ptrs[2], np.uint64, cap)
        b = arr(ptrs[3], np.int32, nb)
        v = arr(ptrs[4], self.np_vt, cap * self.dim).reshape(cap, self.dim)
        return d, k, s, b, v


def murmur3(k):
    return int(lib().hkvo_murmur3(k))


def global_idx(h, cap):
    return int(lib().hkvo_global_idx(h, cap))
