"""The C++ host interface (include/velurex_hip.hpp): the reference's TernaryGemvLayer trait (quintrit-runtime/src/
layer.rs:72-87) and the kernel level of its C++ wrapper (quintrit-c/include/quintrit.hpp:146-191) over the C ABI,
exercised by tests/cpp/test_layer.cpp in the manner of the reference's own C++ test (quintrit-c/tests/cpp/
test_kernel.cpp). The program is built with the library (tests/cpp/Makefile, run by build()); without a device it runs
the checks that need none (ABI, layout, argument errors, the owning class's traits), with one it multiplies against a
brute-force product at the reference's test shapes and extreme fills.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "test_layer")


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(HERE, "cpp")], check=True, capture_output=True)
    return BIN


def test_cpp_interface_without_device():
    r = subprocess.run([_binary(), "--cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "C++ test (no device) passed" in r.stdout


@pytest.mark.gpu
def test_cpp_interface_on_the_gpu():
    print("[cpp] tests/cpp/test_layer", flush=True)
    r = subprocess.run([_binary()], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "C++ test passed" in r.stdout
