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
