"""The no-allocation GEMM entry point (vx_gemm_i32_noalloc_dev) through the C ABI: the same int32 results as
vx_gemm_i32_dev with a caller workspace, bit for bit, on consecutive calls that reuse the library's per-GPU scratch
(the second call smaller than the first, so stale contents of the first stay in the array), and a clear error when a
call would need more workspace than the scratch holds."""
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


def _stream(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def gemm_with_workspace(torch, layer, xd, m, y):
    from quintrit_amd import _lib
    L = _lib.lib()
    rows, cols = layer.shape()
    n = ctypes.c_size_t()
    _lib.check(L.vx_gemm_workspace_bytes(layer.handle, m, ctypes.byref(n)))
    ws = torch.empty(n.value + 256, dtype=torch.uint8, device="cuda")
    base = (ws.data_ptr() + 255) // 256 * 256
    _lib.check(L.vx_gemm_i32_dev(layer.handle, ctypes.c_void_p(xd.data_ptr()), m, cols, ctypes.c_void_p(y.data_ptr()),
                                 rows, ctypes.c_void_p(base), n.value, _stream(torch)))
    torch.cuda.synchronize()
    return n.value


def gemm_noalloc(torch, layer, xd, m, y):
    from quintrit_amd import _lib
    L = _lib.lib()
    rows, cols = layer.shape()
    _lib.check(L.vx_gemm_i32_noalloc_dev(layer.handle, ctypes.c_void_p(xd.data_ptr()), m, cols,
                                         ctypes.c_void_p(y.data_ptr()), rows, _stream(torch)))
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,cols,m", [(3072, 3072, 64), (23040, 3072, 256)])
def test_noalloc_captured_in_a_graph(torch_dev, oracle, rows, cols, m):
    """The entry point for callers under graph capture, captured (the first test of this file, so in a full run the
    call that looks the scratch up runs inside the capture) and replayed three times with new activations and eager
    work in between; every replay equals vx_gemm_i32_dev on the same inputs bit for bit. Two shapes: the small-M path
    (3072 x 3072, 64 tokens) and the staged path (23040 x 3072, 256 tokens)."""
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    t = oracle.gen_trits(0x7C + rows, (rows, cols))
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    rng = np.random.default_rng(rows + m)
    try:
        xd = torch.zeros((m, cols), dtype=torch.int8, device="cuda")
        got = torch.full((m, rows), -9, dtype=torch.int32, device="cuda")
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        print(f"[noalloc graph] capture {rows}x{cols} m={m}", flush=True)
        with torch.cuda.graph(g, stream=side):
            _lib.check(L.vx_gemm_i32_noalloc_dev(layer.handle, ctypes.c_void_p(xd.data_ptr()), m, cols,
                                                 ctypes.c_void_p(got.data_ptr()), rows, _stream(torch)))
        torch.cuda.synchronize()
        for rep in range(3):
            x = rng.integers(-128, 128, size=(m, cols), dtype=np.int8)
            xd.copy_(torch.from_numpy(x))
            want = torch.full((m, rows), -5, dtype=torch.int32, device="cuda")
            gemm_with_workspace(torch, layer, xd, m, want)
            torch.cuda.synchronize()
            print(f"[noalloc graph] replay {rep}", flush=True)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(got, want), rep
            got.fill_(-9)  # eager work between replays
            torch.cuda.synchronize()
        del g
    finally:
        layer.close()


@pytest.mark.parametrize("rows,cols,m1,m2", [(3072, 23040, 128, 8), (23040, 3072, 512, 33), (2560, 2560, 64, 3)])
def test_noalloc_equals_workspace_gemm_twice(torch_dev, oracle, rows, cols, m1, m2):
    """Two calls in a row on one matrix, the second with fewer tokens, each against vx_gemm_i32_dev on the same
    inputs; sampled rows also against the brute-force product."""
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    t = oracle.gen_trits(0x7A + rows + cols, (rows, cols))
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    rng = np.random.default_rng(rows ^ cols)
    try:
        for m in (m1, m2):
            print(f"[noalloc] {rows}x{cols} m={m}", flush=True)
            x = rng.integers(-128, 128, size=(m, cols), dtype=np.int8)
            xd = torch.from_numpy(x).cuda()
            want = torch.full((m, rows), -5, dtype=torch.int32, device="cuda")
            got = torch.full((m, rows), -9, dtype=torch.int32, device="cuda")
            need = gemm_with_workspace(torch, layer, xd, m, want)
            assert need <= 64 << 20
            gemm_noalloc(torch, layer, xd, m, got)
            g, w = got.cpu().numpy(), want.cpu().numpy()
            assert np.array_equal(g, w), m
            sample = rng.choice(rows, size=min(rows, 16), replace=False)
            assert np.array_equal(g[:, sample].astype(np.int64), x.astype(np.int64) @ t[sample].astype(np.int64).T), m
    finally:
        layer.close()


def test_noalloc_rejects_more_than_the_scratch(torch_dev, oracle):
    """A call whose workspace exceeds the scratch (512 tokens of 131072 columns: 67 MB of staged activations) is
    refused with VX_ERR_INVALID_SHAPE before any launch; full-size buffers are passed all the same."""
    from quintrit_amd import VelurexHipLayer
    from quintrit_amd import _lib
    torch = torch_dev
    L = _lib.lib()
    rows, cols, m = 64, 131072, 512
    t = oracle.gen_trits(0x7B, (rows, cols))
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    try:
        n = ctypes.c_size_t()
        _lib.check(L.vx_gemm_workspace_bytes(layer.handle, m, ctypes.byref(n)))
        assert n.value > 64 << 20
        xd = torch.zeros((m, cols), dtype=torch.int8, device="cuda")
        y = torch.zeros((m, rows), dtype=torch.int32, device="cuda")
        st = L.vx_gemm_i32_noalloc_dev(layer.handle, ctypes.c_void_p(xd.data_ptr()), m, cols,
                                       ctypes.c_void_p(y.data_ptr()), rows, _stream(torch))
        assert st == 3
        assert b"no-allocation" in L.vx_last_error_message()
        torch.cuda.synchronize()
    finally:
        layer.close()
