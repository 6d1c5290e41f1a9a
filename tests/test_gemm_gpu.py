"""GPU parity of the batched ternary GEMM (vx_gemm_i32_dev, MFMA i8) through the C ABI.

The reference has no multi-token kernel; its prefill calls the GEMV once per token (quintrit-runtime/src/engine.rs:
625-631), so the GEMM must equal M independent GEMVs bit for bit. Small shapes are checked against brute force; the
BASELINE.json configs[2] shapes (W 23040 x 3072 and 3072 x 23040, M in {8, 32, 128, 512}) against a float64 brute
force of every output.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def gemm(torch, layer, x, ldx=None):
    from quintrit_amd import _lib
    L = _lib.lib()
    rows, cols = layer.shape()
    m = x.shape[0]
    ldx = ldx or cols
    xd = torch.zeros((m, ldx), dtype=torch.int8, device="cuda")
    xd[:, :cols] = torch.from_numpy(x).cuda()
    y = torch.full((m, rows), -7, dtype=torch.int32, device="cuda")
    n = ctypes.c_size_t()
    _lib.check(L.vx_gemm_workspace_bytes(layer.handle, m, ctypes.byref(n)))
    ws = torch.empty(n.value + 256, dtype=torch.uint8, device="cuda")
    base = (ws.data_ptr() + 255) // 256 * 256
    _lib.check(L.vx_gemm_i32_dev(layer.handle, ctypes.c_void_p(xd.data_ptr()), m, ldx, ctypes.c_void_p(y.data_ptr()),
                                 rows, ctypes.c_void_p(base), n.value,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("rows,cols,m", [(64, 160, 1), (1, 1, 3), (65, 161, 13), (130, 3072, 8), (1100, 321, 17),
                                         (200, 4096, 33), (3, 23040, 5), (1024, 3072, 64), (70, 2560, 100),
                                         (300, 6912, 40), (64, 23040, 64), (129, 1, 63), (65, 3200, 65),
                                         (1100, 6913, 97), (8192, 321, 128), (8193, 320, 128)])
def test_gemm_equals_bruteforce(torch_dev, oracle, rows, cols, m):
    from quintrit_amd import VelurexHipLayer
    print(f"[gemm bruteforce] {rows}x{cols} m={m}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols * 3 + m)
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    x = rng.integers(-128, 128, size=(m, cols), dtype=np.int8)
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    got = gemm(torch_dev, layer, x, ldx=cols + (cols % 3))
    want = (x.astype(np.float64) @ t.astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got.astype(np.int64), want)
    layer.close()


def test_gemm_extreme_values(torch_dev, oracle):
    """All +1 / -1 weights times -128 / 127 activations: the largest magnitudes the int32 sums reach."""
    from quintrit_amd import VelurexHipLayer
    rows, cols, m = 64, 23040, 4
    for tv in (1, -1):
        t = np.full((rows, cols), tv, np.int8)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
        x = np.stack([np.full(cols, -128, np.int8), np.full(cols, 127, np.int8),
                      np.where(np.arange(cols) % 2 == 0, 127, -128).astype(np.int8), np.zeros(cols, np.int8)])
        got = gemm(torch_dev, layer, x)
        want = (x.astype(np.int64) @ t.astype(np.int64).T)
        assert np.array_equal(got.astype(np.int64), want)
        layer.close()


@pytest.mark.parametrize("rows,cols", [(23040, 3072), (3072, 23040)])
def test_gemm_config2_equals_bruteforce(torch_dev, oracle, rows, cols):
    """i.i.d. trits (P(-1)=P(+1)=0.35), X quantized per token from N(0,1). Every output of
    every M is compared with a float64 BLAS product of the unpacked trits, which is exact here: the operands are
    integers and every partial sum is at most 128 * 23040 < 2^53 in magnitude."""
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    t = oracle.gen_trits(0xC2 + rows, (rows, cols))
    tf = t.astype(np.float64)
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    rng = np.random.default_rng(rows)
    for m in (8, 32, 48, 64, 128, 512):
        print(f"[gemm config2] {rows}x{cols} m={m}", flush=True)
        x = np.stack([oracle.quantize_i8(rng.standard_normal(cols).astype(np.float32))[0] for _ in range(m)])
        got = gemm(torch, layer, x)
        want = x.astype(np.float64) @ tf.T
        assert np.array_equal(got.astype(np.float64), want), m
    # one token through the GEMV as well: the two kernels agree
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    layer.gemv_i32(torch.from_numpy(x[5]).cuda(), out)
    assert np.array_equal(out.cpu().numpy(), got[5])
    layer.close()
