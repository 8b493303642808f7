"""Python mirror of npu::hkv::HashTable over the gfx950 C ABI (libhkv_amd.so).

Method names, argument order, defaults and error behaviour follow the
reference's HashTable (include/hkv_hashtable.h:895-3485).  Batch arguments
are device buffers: torch tensors on a ROCm device (their data_ptr() is
passed through) or raw integer device addresses.  `stream` is a
torch.cuda.Stream, a raw hipStream_t integer, or None/0 for the null stream.

There is no CPU fallback: importing this module loads the HIP library and
fails if it has not been built (python hierarchicalkv-ascend_amd/build.py).
"""
import ctypes
import dataclasses
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libhkv_amd.so")

HKV_OK, HKV_ERR_INVALID, HKV_ERR_RUNTIME, HKV_ERR_UNSUPPORTED, HKV_ERR_DEVICE = range(5)


# Built-in predicates of erase_if / size_if / export_batch_if (the C++
# facade takes device functors instead).
PRED_SCORE_LT = 0             # score < threshold
PRED_SCORE_GE = 1             # score >= threshold
PRED_SCORE_GT = 2             # score > threshold
PRED_KEY_MASK_EQ = 3          # (key & pattern) == pattern
PRED_KEY_LOW7_GT_SCORE_GT = 4  # (key & 0x7f) > pattern and score > threshold


class EvictStrategy:
    """include/hkv_hashtable.h:111-119"""
    kLru = 0
    kLfu = 1
    kEpochLru = 2
    kEpochLfu = 3
    kCustomized = 4


KEY_TYPES = {"u64": 0, "uint64": 0, "i64": 1, "int64": 1}
VALUE_TYPES = {"f32": 0, "float32": 0, "f64": 1, "float64": 1, "f16": 2,
               "float16": 2, "bf16": 3, "bfloat16": 3, "i8": 4, "int8": 4,
               "u8": 5, "uint8": 5, "i16": 6, "int16": 6, "u16": 7,
               "uint16": 7, "i32": 8, "int32": 8, "u32": 9, "uint32": 9,
               "i64": 10, "int64": 10, "u64": 11, "uint64": 11}
IGNORED_GLOBAL_EPOCH = 0xFFFFFFFFFFFFFFFF


class HkvException(RuntimeError):
    """Argument/option check failure (reference include/debug.h:53-74)."""


class NpuException(RuntimeError):
    """Device runtime failure (reference include/debug.h:30-51)."""


class UnsupportedError(RuntimeError):
    """Feature not available in this build."""


@dataclasses.dataclass
class HashTableOptions:
    """Field-for-field include/hashtable_options.h:33-65."""
    init_capacity: int = 0
    max_capacity: int = 0
    max_hbm_for_vectors: int = 0
    max_bucket_size: int = 128
    dim: int = 64
    max_load_factor: float = 0.5
    block_size: int = 128
    io_block_size: int = 1024
    device_id: int = -1
    io_by_cpu: bool = False
    use_constant_memory: bool = False
    reserved_key_start_bit: int = 0
    num_of_buckets_per_alloc: int = 1
    api_lock: bool = False


class _COptions(ctypes.Structure):
    _fields_ = [("init_capacity", ctypes.c_uint64),
                ("max_capacity", ctypes.c_uint64),
                ("max_hbm_for_vectors", ctypes.c_uint64),
                ("max_bucket_size", ctypes.c_uint64),
                ("dim", ctypes.c_uint64),
                ("max_load_factor", ctypes.c_float),
                ("block_size", ctypes.c_int32),
                ("io_block_size", ctypes.c_int32),
                ("device_id", ctypes.c_int32),
                ("io_by_cpu", ctypes.c_int32),
                ("use_constant_memory", ctypes.c_int32),
                ("reserved_key_start_bit", ctypes.c_int32),
                ("num_of_buckets_per_alloc", ctypes.c_uint64),
                ("api_lock", ctypes.c_int32)]


_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGS = {
    "hkv_options_default": [_vp],
    "hkv_create": [_vp, _i32, _i32, _i32, _vp],
    "hkv_destroy": [_vp],
    "hkv_insert_or_assign": [_vp, _u64, _vp, _vp, _vp, _vp, _i32, _i32],
    "hkv_insert_or_assign_noalloc": [_vp, _u64, _vp, _vp, _vp, _vp, _i32, _i32],
    "hkv_insert_and_evict": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp, _i32, _i32],
    "hkv_accum_or_assign": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _i32],
    "hkv_find_or_insert": [_vp, _u64, _vp, _vp, _vp, _vp, _i32, _i32],
    "hkv_assign_scores": [_vp, _u64, _vp, _vp, _vp, _i32],
    "hkv_find": [_vp, _u64, _vp, _vp, _vp, _vp, _vp],
    "hkv_find_missed": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "hkv_assign": [_vp, _u64, _vp, _vp, _vp, _vp, _i32],
    "hkv_assign_values": [_vp, _u64, _vp, _vp, _vp, _i32],
    "hkv_contains": [_vp, _u64, _vp, _vp, _vp],
    "hkv_erase_if": [_vp, _i32, _u64, _u64, _vp, ctypes.POINTER(_u64)],
    "hkv_size_if": [_vp, _i32, _u64, _u64, _vp, _vp],
    "hkv_export_batch_if": [_vp, _i32, _u64, _u64, _u64, _u64, _vp, _vp, _vp, _vp,
                            _vp],
    "hkv_set_max_capacity": [_vp, _u64],
    "hkv_device_view_get": [_vp, _vp],
    "hkv_find_ptr": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _i32],
    "hkv_find_and_update": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _i32],
    "hkv_find_or_insert_ptr": [_vp, _u64, _vp, _vp, _vp, _vp, _vp, _i32, _i32,
                               _vp],
    "hkv_lock_keys": [_vp, _u64, _vp, _vp, _vp, _vp, _vp],
    "hkv_unlock_keys": [_vp, _u64, _vp, _vp, _vp, _vp],
    "hkv_slot_addresses": [_vp, _u64, _vp, _vp, _vp],
    "hkv_erase": [_vp, _u64, _vp, _vp],
    "hkv_clear": [_vp, _vp],
    "hkv_export_batch": [_vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp],
    "hkv_reserve": [_vp, _u64, _vp],
    "hkv_set_global_epoch": [_vp, _u64],
    "hkv_size": [_vp, _vp, _vp],
    "hkv_load_factor": [_vp, _vp, _vp],
    "hkv_capacity": [_vp],
    "hkv_dim": [_vp],
    "hkv_max_bucket_size": [_vp],
    "hkv_bucket_count": [_vp],
    "hkv_is_pure_hbm_mode": [_vp],
    "hkv_last_error": [],
    "hkv_set_lru_clock": [_vp, _u64, _i32],
    "hkv_live_count": [_vp, _vp, ctypes.POINTER(_u64)],
    "hkv_save": [_vp, _vp, _vp, _u64, _vp, ctypes.POINTER(_u64)],
    "hkv_load": [_vp, _vp, _vp, _u64, _vp, ctypes.POINTER(_u64)],
    "hkv_local_kv_file_open": [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                               ctypes.c_char_p],
    "hkv_local_kv_file_close": [_vp],
    "hkv_local_kv_file_write": [_vp, _u64, _u64, _vp, _vp, _vp],
    "hkv_local_kv_file_read": [_vp, _u64, _u64, _vp, _vp, _vp],
}
# Callback types of hkv_save / hkv_load (a key-value file's write and read).
_KV_FN = ctypes.CFUNCTYPE(_u64, _vp, _u64, _u64, _vp, _vp, _vp)
_RESTYPES = {"hkv_options_default": None, "hkv_capacity": _u64, "hkv_dim": _u64,
             "hkv_max_bucket_size": _u64, "hkv_bucket_count": _u64,
             "hkv_last_error": ctypes.c_char_p, "hkv_local_kv_file_open": _vp,
             "hkv_local_kv_file_close": None, "hkv_local_kv_file_write": _u64,
             "hkv_local_kv_file_read": _u64}

EXPORTED_SYMBOLS = tuple(_SIGS)


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise ImportError(
            "libhkv_amd.so is not built; run python "
            "hierarchicalkv-ascend_amd/build.py (no CPU fallback exists)")
    # One process must use one HIP runtime.  torch bundles its own
    # libamdhip64 (soname libamdhip64.so.7); loading torch first makes
    # libhkv_amd.so bind to that same runtime by soname instead of pulling
    # a second copy from /opt/rocm, which would not see the GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, args in _SIGS.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = _RESTYPES.get(name, _i32)
    return lib


_LIB = load_library()


def _check(rc):
    if rc == HKV_OK:
        return
    msg = (_LIB.hkv_last_error() or b"").decode(errors="replace")
    if rc == HKV_ERR_INVALID:
        raise HkvException(msg)
    if rc == HKV_ERR_RUNTIME:
        raise RuntimeError(msg)
    if rc == HKV_ERR_UNSUPPORTED:
        raise UnsupportedError(msg)
    raise NpuException(msg)


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(s):
    if s is None or s == 0:
        return None
    if isinstance(s, int):
        return s
    return s.cuda_stream


class BaseKVFile:
    """Key-value file of save/load (include/types.h:291-330).  Subclasses
    implement read and write over numpy arrays: read fills up to n records
    and returns the count, write stores n records and returns the count."""

    def read(self, n, dim, keys, values, scores):
        raise NotImplementedError

    def write(self, n, dim, keys, values, scores):
        raise NotImplementedError


class LocalKVFile(BaseKVFile):
    """Three raw files: keys (u64), rows (dim values each), scores (u64)
    (include/types.h:350-464); read and write run in the library."""

    def __init__(self):
        self._f = None

    def open(self, keys_path, values_path, scores_path, mode):
        self.close()
        self._f = _LIB.hkv_local_kv_file_open(os.fsencode(keys_path), os.fsencode(values_path),
                                              os.fsencode(scores_path), mode.encode())
        return bool(self._f)

    def close(self):
        if self._f:
            _LIB.hkv_local_kv_file_close(self._f)
        self._f = None

    def __del__(self):
        if _LIB is not None:
            self.close()


_NP_VALUE = {0: "float32", 1: "float64", 2: "float16", 3: "uint16", 4: "int8", 5: "uint8",
             6: "int16", 7: "uint16", 8: "int32", 9: "uint32", 10: "int64", 11: "uint64"}


class HashTable:
    """HashTable<K, V, S=uint64_t, Strategy> with runtime K/V/Strategy."""

    def __init__(self, key_type="u64", value_type="f32",
                 strategy=EvictStrategy.kLru):
        self.key_type = KEY_TYPES[key_type]
        self.value_type = VALUE_TYPES[value_type]
        self.evict_strategy = strategy
        self._h = None

    def init(self, options):
        if self._h is not None:
            return
        o = _COptions()
        for f in HashTableOptions.__dataclass_fields__:
            setattr(o, f, int(getattr(options, f)) if f != "max_load_factor"
                    else float(getattr(options, f)))
        h = ctypes.c_void_p()
        _check(_LIB.hkv_create(ctypes.byref(o), self.key_type,
                               self.value_type, self.evict_strategy,
                               ctypes.byref(h)))
        self._h = h
        self.options = options

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _LIB is not None:
            _LIB.hkv_destroy(h)
            self._h = None

    # --- insert-like ---------------------------------------------------------
    def insert_or_assign(self, n, keys, values, scores=None, stream=0,
                         unique_key=True, ignore_evict_strategy=False):
        _check(_LIB.hkv_insert_or_assign(self._h, n, _ptr(keys), _ptr(values),
                                         _ptr(scores), _stream(stream),
                                         int(unique_key),
                                         int(ignore_evict_strategy)))

    def insert_or_assign_noalloc(self, n, keys, values, scores=None, stream=0,
                                 unique_key=True, ignore_evict_strategy=False):
        """insert_or_assign that allocates no device memory (no counterpart
        in the reference; for callers that cannot allocate).  Needs a table
        at its maximum capacity and a batch whose scratch fits the library's
        64 MiB static array; otherwise raises HkvException."""
        _check(_LIB.hkv_insert_or_assign_noalloc(self._h, n, _ptr(keys), _ptr(values),
                                                 _ptr(scores), _stream(stream),
                                                 int(unique_key),
                                                 int(ignore_evict_strategy)))

    def insert_and_evict(self, n, keys, values, scores, evicted_keys,
                         evicted_values, evicted_scores,
                         d_evicted_counter=None, stream=0, unique_key=True,
                         ignore_evict_strategy=False):
        """With `d_evicted_counter` the count accumulates on the device;
        without it the call synchronizes and returns the count
        (include/hkv_hashtable.h:1260-1396)."""
        if d_evicted_counter is not None:
            _check(_LIB.hkv_insert_and_evict(
                self._h, n, _ptr(keys), _ptr(values), _ptr(scores),
                _ptr(evicted_keys), _ptr(evicted_values), _ptr(evicted_scores),
                _ptr(d_evicted_counter), _stream(stream), int(unique_key),
                int(ignore_evict_strategy)))
            return None
        import torch
        if n == 0:
            return 0
        cnt = torch.zeros(1, dtype=torch.int64, device=keys.device)
        _check(_LIB.hkv_insert_and_evict(
            self._h, n, _ptr(keys), _ptr(values), _ptr(scores),
            _ptr(evicted_keys), _ptr(evicted_values), _ptr(evicted_scores),
            _ptr(cnt), _stream(stream), int(unique_key),
            int(ignore_evict_strategy)))
        return int(cnt.item())

    def accum_or_assign(self, n, keys, value_or_deltas, accum_or_assigns,
                        scores=None, stream=0, ignore_evict_strategy=False):
        _check(_LIB.hkv_accum_or_assign(self._h, n, _ptr(keys),
                                        _ptr(value_or_deltas),
                                        _ptr(accum_or_assigns), _ptr(scores),
                                        _stream(stream),
                                        int(ignore_evict_strategy)))

    def find_or_insert(self, n, keys, values, scores=None, stream=0,
                       unique_key=True, ignore_evict_strategy=False):
        _check(_LIB.hkv_find_or_insert(self._h, n, _ptr(keys), _ptr(values),
                                       _ptr(scores), _stream(stream),
                                       int(unique_key),
                                       int(ignore_evict_strategy)))

    def assign_scores(self, n, keys, scores=None, stream=0, unique_key=True):
        _check(_LIB.hkv_assign_scores(self._h, n, _ptr(keys), _ptr(scores),
                                      _stream(stream), int(unique_key)))

    def assign(self, n, keys, values, scores=None, stream=0, unique_key=True):
        """include/hkv_hashtable.h:1830-1921."""
        _check(_LIB.hkv_assign(self._h, n, _ptr(keys), _ptr(values), _ptr(scores),
                               _stream(stream), int(unique_key)))

    def assign_values(self, n, keys, values, stream=0, unique_key=True):
        """include/hkv_hashtable.h:2003-2093."""
        _check(_LIB.hkv_assign_values(self._h, n, _ptr(keys), _ptr(values),
                                      _stream(stream), int(unique_key)))

    # --- lookups -------------------------------------------------------------
    def contains(self, n, keys, founds, stream=0):
        """include/hkv_hashtable.h:2330-2347."""
        _check(_LIB.hkv_contains(self._h, n, _ptr(keys), _ptr(founds),
                                 _stream(stream)))

    def find(self, n, keys, values, founds, scores=None, stream=0):
        _check(_LIB.hkv_find(self._h, n, _ptr(keys), _ptr(values),
                             _ptr(founds), _ptr(scores), _stream(stream)))

    def find_missed(self, n, keys, values, missed_keys, missed_indices,
                    missed_size, scores=None, stream=0):
        """The missed-keys overload of find (include/hkv_hashtable.h:2175)."""
        _check(_LIB.hkv_find_missed(self._h, n, _ptr(keys), _ptr(values),
                                    _ptr(missed_keys), _ptr(missed_indices),
                                    _ptr(missed_size), _ptr(scores),
                                    _stream(stream)))

    # --- pointer APIs --------------------------------------------------------
    # The reference overloads find / find_or_insert on `V**`; here the
    # pointer forms have their own names.  Address arrays are uint64/int64
    # tensors of n entries (0 = null).
    def find_ptr(self, n, keys, values, founds=None, scores=None, stream=0,
                 unique_key=True):
        """find, pointer overload (include/hkv_hashtable.h:2244-2262)."""
        _check(_LIB.hkv_find_ptr(self._h, n, _ptr(keys), _ptr(values),
                                 _ptr(founds), _ptr(scores), _stream(stream),
                                 int(unique_key)))

    def find_and_update(self, n, keys, values, founds=None, scores=None,
                        stream=0, unique_key=True):
        """include/hkv_hashtable.h:2288-2317; scores are input and output."""
        _check(_LIB.hkv_find_and_update(self._h, n, _ptr(keys), _ptr(values),
                                        _ptr(founds), _ptr(scores),
                                        _stream(stream), int(unique_key)))

    def find_or_insert_ptr(self, n, keys, values, founds, scores=None, stream=0,
                           unique_key=True, ignore_evict_strategy=False,
                           locked_key_ptrs=None):
        """find_or_insert, pointer overload (include/hkv_hashtable.h:1658-1728)."""
        _check(_LIB.hkv_find_or_insert_ptr(self._h, n, _ptr(keys), _ptr(values),
                                           _ptr(founds), _ptr(scores),
                                           _stream(stream), int(unique_key),
                                           int(ignore_evict_strategy),
                                           _ptr(locked_key_ptrs)))

    def lock_keys(self, n, keys, locked_key_ptrs, success=None, stream=0,
                  scores=None):
        """include/hkv_hashtable.h:1744-1771."""
        _check(_LIB.hkv_lock_keys(self._h, n, _ptr(keys), _ptr(locked_key_ptrs),
                                  _ptr(success), _stream(stream), _ptr(scores)))

    def unlock_keys(self, n, locked_key_ptrs, keys, success=None, stream=0):
        """include/hkv_hashtable.h:1788-1804."""
        _check(_LIB.hkv_unlock_keys(self._h, n, _ptr(locked_key_ptrs),
                                    _ptr(keys), _ptr(success), _stream(stream)))

    def slot_addresses(self, slots):
        """Test hook: (key word, value row) addresses of global slots, as
        numpy uint64 arrays (no device work)."""
        import numpy as np
        sl = np.ascontiguousarray(slots, dtype=np.uint64)
        kp = np.zeros(sl.size, np.uint64)
        vp = np.zeros(sl.size, np.uint64)
        _check(_LIB.hkv_slot_addresses(self._h, sl.size, sl.ctypes.data,
                                       kp.ctypes.data, vp.ctypes.data))
        return kp, vp

    # --- predicates (built-in predicate kinds, PRED_*) ------------------------
    def erase_if(self, pred, pattern, threshold, stream=0):
        """include/hkv_hashtable.h:2409-2441; returns the number erased."""
        out = ctypes.c_uint64()
        _check(_LIB.hkv_erase_if(self._h, pred, pattern, threshold, _stream(stream),
                                 ctypes.byref(out)))
        return out.value

    def size_if(self, pred, pattern, threshold, d_counter, stream=0):
        """include/hkv_hashtable.h:2829-2845; the count lands in d_counter."""
        _check(_LIB.hkv_size_if(self._h, pred, pattern, threshold, _ptr(d_counter),
                                _stream(stream)))

    def export_batch_if(self, pred, pattern, threshold, n, offset, d_counter, keys,
                        values, scores=None, stream=0):
        """include/hkv_hashtable.h:2623-2672; tuple order is unspecified."""
        _check(_LIB.hkv_export_batch_if(self._h, pred, pattern, threshold, n, offset,
                                        _ptr(d_counter), _ptr(keys), _ptr(values),
                                        _ptr(scores), _stream(stream)))

    def empty(self, stream=0):
        return self.size(stream) == 0

    def set_max_capacity(self, new_max_capacity):
        """include/hkv_hashtable.h:2955-2977."""
        _check(_LIB.hkv_set_max_capacity(self._h, new_max_capacity))

    # --- maintenance ---------------------------------------------------------
    def erase(self, n, keys, stream=0):
        _check(_LIB.hkv_erase(self._h, n, _ptr(keys), _stream(stream)))

    def clear(self, stream=0):
        _check(_LIB.hkv_clear(self._h, _stream(stream)))

    def export_batch(self, n, offset, keys, values, scores=None,
                     d_counter=None, stream=0):
        """With `d_counter` the count is left on the device; without it the
        call synchronizes and returns the count."""
        if d_counter is not None:
            _check(_LIB.hkv_export_batch(self._h, n, offset, _ptr(d_counter),
                                         _ptr(keys), _ptr(values),
                                         _ptr(scores), _stream(stream)))
            return None
        import torch
        cnt = torch.zeros(1, dtype=torch.int64, device=keys.device)
        _check(_LIB.hkv_export_batch(self._h, n, offset, _ptr(cnt), _ptr(keys),
                                     _ptr(values), _ptr(scores),
                                     _stream(stream)))
        return int(cnt.item())

    def _kv_callbacks(self, file):
        if isinstance(file, LocalKVFile):
            if not file._f:
                raise HkvException("the key-value file is not open")
            return (ctypes.cast(_LIB.hkv_local_kv_file_write, _KV_FN),
                    ctypes.cast(_LIB.hkv_local_kv_file_read, _KV_FN), file._f)
        import numpy as np
        vt = np.dtype(_NP_VALUE[self.value_type])

        def arrays(n, row_bytes, k, v, s):
            dim = row_bytes // vt.itemsize
            ka = np.ctypeslib.as_array(ctypes.cast(k, ctypes.POINTER(ctypes.c_uint64)), (n,))
            va = np.ctypeslib.as_array(ctypes.cast(v, ctypes.POINTER(ctypes.c_uint8)),
                                       (n * row_bytes,)).view(vt).reshape(n, dim)
            sa = np.ctypeslib.as_array(ctypes.cast(s, ctypes.POINTER(ctypes.c_uint64)), (n,))
            return dim, ka, va, sa

        def w(ctx, n, row_bytes, k, v, s):
            if n == 0:
                return 0
            dim, ka, va, sa = arrays(n, row_bytes, k, v, s)
            return int(file.write(n, dim, ka, va, sa))

        def r(ctx, n, row_bytes, k, v, s):
            dim, ka, va, sa = arrays(n, row_bytes, k, v, s)
            return int(file.read(n, dim, ka, va, sa))
        return _KV_FN(w), _KV_FN(r), None

    def save(self, file, max_workspace_size=1 << 20, stream=0):
        """include/hkv_hashtable.h:3021-3118; returns the records written."""
        w, _r, ctx = self._kv_callbacks(file)
        out = _u64(0)
        _check(_LIB.hkv_save(self._h, ctypes.cast(w, _vp), ctx, max_workspace_size,
                             _stream(stream), ctypes.byref(out)))
        return out.value

    def load(self, file, max_workspace_size=1 << 20, stream=0):
        """include/hkv_hashtable.h:3134-3195; returns the records read."""
        _w, r, ctx = self._kv_callbacks(file)
        out = _u64(0)
        _check(_LIB.hkv_load(self._h, ctypes.cast(r, _vp), ctx, max_workspace_size,
                             _stream(stream), ctypes.byref(out)))
        return out.value

    def reserve(self, new_capacity, stream=0):
        _check(_LIB.hkv_reserve(self._h, new_capacity, _stream(stream)))

    def set_global_epoch(self, epoch):
        _check(_LIB.hkv_set_global_epoch(self._h, epoch))

    def size(self, stream=0):
        out = ctypes.c_uint64()
        _check(_LIB.hkv_size(self._h, _stream(stream), ctypes.byref(out)))
        return out.value

    def load_factor(self, stream=0):
        out = ctypes.c_float()
        _check(_LIB.hkv_load_factor(self._h, _stream(stream),
                                    ctypes.byref(out)))
        return out.value

    def capacity(self):
        return int(_LIB.hkv_capacity(self._h))

    def dim(self):
        return int(_LIB.hkv_dim(self._h))

    def max_bucket_size(self):
        return int(_LIB.hkv_max_bucket_size(self._h))

    def bucket_count(self):
        return int(_LIB.hkv_bucket_count(self._h))

    def is_pure_hbm_mode(self):
        return bool(_LIB.hkv_is_pure_hbm_mode(self._h))

    # --- test hook -----------------------------------------------------------
    def set_lru_clock(self, clock, enable=True):
        """Fixes the Lru/EpochLru clock (no reference counterpart)."""
        _check(_LIB.hkv_set_lru_clock(self._h, clock, int(enable)))

    def live_count(self, stream=0):
        """Live-key count kept on the device (no reference counterpart)."""
        out = _u64(0)
        _check(_LIB.hkv_live_count(self._h, _stream(stream), ctypes.byref(out)))
        return out.value
