"""CPU-only checks of the C-ABI library: it loads, exports every symbol that
include/hkv_amd.h declares, and rejects invalid options on the host before
touching a device (the reference's init checks, hkv_hashtable.h:991-1024)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "hierarchicalkv-ascend_amd", "lib", "libhkv_amd.so")
HDR = os.path.join(ROOT, "include", "hkv_amd.h")

pytestmark = pytest.mark.skipif(not os.path.exists(LIB),
                                reason="libhkv_amd.so not built")


def declared_symbols():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hkv_[a-z_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib, s), s


def test_python_mirror_binds_every_symbol():
    import hkv_amd
    assert sorted(hkv_amd.EXPORTED_SYMBOLS) == declared_symbols()


def _opts(**kw):
    import hkv_amd
    o = hkv_amd.HashTableOptions(init_capacity=1 << 12, max_capacity=1 << 12,
                                 max_hbm_for_vectors=1 << 30, dim=8)
    for k, v in kw.items():
        setattr(o, k, v)
    return o


@pytest.mark.parametrize("kw,exc", [
    (dict(max_bucket_size=8), "HkvException"),
    (dict(max_bucket_size=100), "HkvException"),
    (dict(num_of_buckets_per_alloc=3), "HkvException"),
    (dict(init_capacity=64), "HkvException"),
    (dict(reserved_key_start_bit=63), "HkvException"),
    (dict(io_by_cpu=True), "HkvException"),
    (dict(io_by_cpu=True, max_hbm_for_vectors=0), "UnsupportedError"),
    (dict(api_lock=True), "UnsupportedError"),
    (dict(max_bucket_size=256), "UnsupportedError"),
])
def test_invalid_options_rejected_on_host(kw, exc):
    import hkv_amd
    t = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kLru)
    with pytest.raises(getattr(hkv_amd, exc)):
        t.init(_opts(**kw))


def test_options_default_matches_reference():
    import hkv_amd
    o = hkv_amd._COptions()
    hkv_amd._LIB.hkv_options_default(ctypes.byref(o))
    d = hkv_amd.HashTableOptions()
    for f in d.__dataclass_fields__:
        v = getattr(o, f)
        if f == "max_load_factor":
            assert abs(v - d.max_load_factor) < 1e-7
        else:
            assert v == int(getattr(d, f)), f


def test_unknown_types_rejected():
    import hkv_amd
    lib = hkv_amd._LIB
    o = hkv_amd._COptions()
    lib.hkv_options_default(ctypes.byref(o))
    o.init_capacity = o.max_capacity = 1 << 12
    h = ctypes.c_void_p()
    assert lib.hkv_create(ctypes.byref(o), 7, 0, 0, ctypes.byref(h)) == 1
    assert lib.hkv_create(ctypes.byref(o), 0, 99, 0, ctypes.byref(h)) == 1
    assert lib.hkv_create(ctypes.byref(o), 0, 0, 9, ctypes.byref(h)) == 1
    assert b"strategy" in lib.hkv_last_error()


def test_cpp_facade_builds_and_links():
    """The header-only npu::hkv::HashTable facade compiles against the C ABI
    and links with libhkv_amd.so (run on a GPU by test_gpu_cpp_facade)."""
    import subprocess
    subprocess.check_call(["bash", os.path.join(ROOT, "tests", "cpp", "build.sh")])
    assert os.path.exists(os.path.join(ROOT, "tests", "cpp", "build", "facade_parity"))
