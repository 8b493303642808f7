"""C++ drop-in check on the GPU: tests/cpp/facade_parity drives the table
through include/hkv_hashtable.hpp (npu::hkv::HashTable) and compares find,
erase and export results with the oracle bit-exactly."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "build", "facade_parity")


@pytest.mark.gpu
def test_cpp_facade_parity():
    if not os.path.exists(BIN):
        pytest.skip("tests/cpp/build/facade_parity not built (tests/cpp/build.sh)")
    out = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(out.stdout, out.stderr)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "facade parity ok" in out.stdout


@pytest.mark.gpu
def test_cpp_facade_functor_apis():
    """erase_if / erase_if_v2 / export_batch_if / export_batch_if_v2 /
    size_if / for_each instantiated with functors written as the
    reference's tests write them (tests/cpp/facade_predicates.hip)."""
    binp = os.path.join(ROOT, "tests", "cpp", "build", "facade_predicates")
    if not os.path.exists(binp):
        pytest.skip("tests/cpp/build/facade_predicates not built (tests/cpp/build.sh)")
    out = subprocess.run([binp], capture_output=True, text=True, timeout=120)
    print(out.stdout, out.stderr)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "facade predicates ok" in out.stdout
