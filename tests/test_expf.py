"""The device expf (quintrit_amd/csrc/vx_expf.h) equals the host's glibc expf on every float.

The reference's attention takes its exponentials from Rust's f32::exp, i.e. glibc's expf (quintrit-runtime/src/
attention.rs:423-462); the GPU must reproduce them bit for bit. This test compiles the header for the CPU and compares
all 2^32 inputs with the host libm (about 10 s on 8 threads). The GPU side of the same function is checked in
tests/test_decode_gpu.py.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r'''
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include "vx_expf.h"
int main() {
    long bad = 0;
#pragma omp parallel for reduction(+:bad) schedule(static, 1 << 20)
    for (long i = 0; i < (1L << 32); ++i) {
        uint32_t u = (uint32_t)i; float x; std::memcpy(&x, &u, 4);
        const float r = expf(x), a = vx::glibc_expf(x);
        uint32_t ur, ua; std::memcpy(&ur, &r, 4); std::memcpy(&ua, &a, 4);
        if (!(ua == ur || (std::isnan(r) && std::isnan(a)))) ++bad;
    }
    std::printf("%ld\n", bad);
    return 0;
}
'''


def test_glibc_expf_on_every_float(tmp_path):
    src = tmp_path / "expf_check.cpp"
    src.write_text(SRC)
    exe = tmp_path / "expf_check"
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c++20", "-I",
                    os.path.join(ROOT, "quintrit_amd", "csrc"), str(src), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.strip()
    assert out == "0", f"{out} floats differ from the host expf"
