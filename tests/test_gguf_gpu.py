"""GPU upload of GGUF ternary tensors (vx_gguf_upload_matrix, vx_matrix_create_ggml_dev): the payload is converted in
HBM into a GEMV matrix. Checked through the exact GEMV: int32 outputs equal brute force over the oracle's trits and the
outputs of the matrix built from the host conversion; the tensor's weight scale reaches the fp32 epilogue."""
import ctypes
import os

import numpy as np
import pytest

from gguf_writer import build

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def payload(oracle, ty, trits, d_bits=0x3800):
    if ty == 36:
        return oracle.i2s_pack(trits)
    return oracle.tq_pack(ty, trits.reshape(-1), d_bits)


@pytest.mark.parametrize("ty", [36, 34, 35])
@pytest.mark.parametrize("rows,cols", [(2, 256), (65, 384), (130, 1280), (96, 3072), (64, 23040)])
def test_upload_equals_brute_force(torch_dev, oracle, tmp_path, ty, rows, cols):
    torch = torch_dev
    from quintrit_amd._lib import check, lib
    from quintrit_amd.gguf import GgufFile
    from quintrit_amd.layer import VelurexHipLayer
    if ty != 36 and rows * cols % 256:
        # a TQ tensor holds whole 256-weight blocks: 65 x 384 is refused before any device work
        from quintrit_amd._lib import VxError
        d = torch.zeros(rows * cols, dtype=torch.uint8, device="cuda")
        h = ctypes.c_void_p()
        with pytest.raises(VxError, match="INVALID_SHAPE"):
            check(lib().vx_matrix_create_ggml_dev(ty, ctypes.c_void_p(d.data_ptr()), d.numel(), rows, cols,
                                                  ctypes.c_float(1.0), ctypes.byref(h)))
        assert not h.value
        return
    rng = np.random.default_rng(rows * 7 + cols + ty)
    trits = rng.integers(-1, 2, (rows, cols)).astype(np.int8)
    data = payload(oracle, ty, trits)
    tail = np.array([0.25], np.float32).tobytes() if ty == 36 else b""
    path = tmp_path / "w.gguf"
    path.write_bytes(build([], [("w", [cols, rows], ty, data.tobytes() + tail)]))
    acts = rng.integers(-128, 128, cols).astype(np.int8)
    want = trits.astype(np.int64) @ acts.astype(np.int64)
    a = torch.from_numpy(acts).cuda()
    with GgufFile(path) as g:
        m = g.upload_matrix("w")
        planar, _, _, scale = g.convert_planar("w")
    assert m.shape() == (rows, cols) and m.weight_scale() == (0.25 if ty == 36 else 0.5) == scale
    host = VelurexHipLayer(planar, rows, cols, scale)
    # the payload already in device memory
    d = torch.from_numpy(data).cuda()
    h = ctypes.c_void_p()
    check(lib().vx_matrix_create_ggml_dev(ty, ctypes.c_void_p(d.data_ptr()), d.numel(), rows, cols,
                                          ctypes.c_float(2.0), ctypes.byref(h)))
    dev = VelurexHipLayer._from_handle(h)
    for layer in (m, host, dev):
        out = torch.empty(rows, dtype=torch.int32, device="cuda")
        layer.gemv_i32(a, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().astype(np.int64), want)
    outf = torch.empty(rows, dtype=torch.float32, device="cuda")
    m.gemv_f32(a, 2.0, outf)
    torch.cuda.synchronize()
    post = np.float32(scale) / np.float32(2.0)
    assert np.array_equal(outf.cpu().numpy(), want.astype(np.float32) * post)
    for layer in (m, host, dev):
        layer.close()


def test_upload_errors(torch_dev, oracle, tmp_path):
    from quintrit_amd._lib import VxError
    from quintrit_amd.gguf import GgufFile
    trits = np.zeros(512, np.int8)
    same = oracle.tq_pack(34, trits, 0x3800)
    differ = same.copy()
    differ[54 + 52] ^= 1
    path = tmp_path / "e.gguf"
    path.write_bytes(build([], [("f", [4, 4], 0, bytes(64)), ("d", [256, 2], 34, differ.tobytes()),
                                ("v", [512], 34, same.tobytes())]))
    with GgufFile(path) as g:
        with pytest.raises(VxError, match="UNSUPPORTED"):
            g.upload_matrix("f")
        with pytest.raises(VxError, match="FORMAT"):
            g.upload_matrix("d")
        with pytest.raises(VxError, match="INVALID_SHAPE"):
            g.upload_matrix("v")


@pytest.mark.parametrize("bs", [64, 128])
def test_q2_0_upload_bit_exact(torch_dev, oracle, tmp_path, bs):
    """A Q2_0 GGUF tensor uploaded as a Q2_0 GEMV matrix (vx_gguf_upload_q2_matrix) gives the oracle's
    dot_row_scalar results (block_scaled.rs:175-202) on the decoded trits and scales, bit for bit, with its lane sums."""
    import ctypes
    from test_gguf import q2_0_payload
    from gguf_writer import build
    from quintrit_amd.gguf import GgufFile
    rng = np.random.default_rng(11 + bs)
    rows, cols = 300, 2560
    data, trits, d = q2_0_payload(rng, rows, cols, bs)
    path = os.path.join(tmp_path, "q2.gguf")
    with open(path, "wb") as f:
        f.write(build([], [("w", [cols, rows], 42, data), ("f", [8], 0, bytes(32))]))
    acts = oracle.gen_i8(5, cols, -127, 127)
    as32 = rng.uniform(0.005, 0.05, cols // 32).astype(np.float32)
    with GgufFile(path) as g:
        mat = g.upload_q2_matrix("w")
    torch = torch_dev
    try:
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        a, s = torch.from_numpy(acts).cuda(), torch.from_numpy(as32).cuda()
        out = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        lanes = torch.empty(rows * (cols // 32) * 8, dtype=torch.int32, device="cuda")
        mat.gemv_f32(a, s, out, stream)
        mat.lane_sums(a, lanes, stream)
        torch.cuda.synchronize()
        planar = oracle.pack_matrix(trits.reshape(rows, cols))
        ws = np.repeat(d, bs // 64).view(np.float16).astype(np.float32)
        want = oracle.q2_0_gemv(planar, ws, acts, as32, rows, cols)
        assert np.array_equal(lanes.cpu().numpy(), oracle.q2_0_lane_sums(planar, acts, rows, cols).reshape(-1))
        assert np.array_equal(out.cpu().numpy().view(np.uint32), np.asarray(want, np.float32).view(np.uint32))
    finally:
        mat.close()
