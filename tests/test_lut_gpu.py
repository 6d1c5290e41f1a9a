"""GPU parity of the compact-table GEMV (vx_compact_lut_dev, vx_gemv_lut_*, vx_lut_plan_create) through the C ABI.

The tables must equal the oracle's restatement of build_compact_wide_impl (quintrit-core/src/simd/avx512.rs:1216-1247)
byte for byte; the products are exact int32 (brute force) and the fp32 outputs equal the digit-table GEMV's bit for
bit. Patterns and shapes follow the reference's GPU tests (quintrit-cuda/tests/gemv.rs:46-64,77-125).
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


def exact_gemv(trits, acts):
    """Brute-force product; float32 BLAS is exact here (|partial sums| < 2^24, integer operands)."""
    return (trits.astype(np.float32) @ acts.astype(np.float32)).astype(np.int64)


def acts_of(kind, cols, rng):
    return {"random": lambda: rng.integers(-128, 128, size=cols, dtype=np.int8),
            "max": lambda: np.full(cols, 127, np.int8),
            "min": lambda: np.full(cols, -128, np.int8),
            "alternating": lambda: np.where(np.arange(cols) % 2 == 0, 127, -128).astype(np.int8)}[kind]()


def gpu_lut(torch, a, cols):
    from quintrit_amd.layer import compact_lut
    lut = compact_lut(torch.from_numpy(a).cuda(), cols)
    torch.cuda.synchronize()
    return lut


@pytest.mark.parametrize("cols", [1, 5, 159, 160, 161, 320, 2560, 3072, 6912, 23040])
def test_tables_equal_the_oracle(torch_dev, oracle, cols):
    print(f"[lut tables] cols={cols}", flush=True)
    rng = np.random.default_rng(cols + 7)
    for kind in ("random", "max", "min", "alternating"):
        a = acts_of(kind, cols, rng)
        got = gpu_lut(torch_dev, a, cols).cpu().numpy()
        want = oracle.build_compact_wide_lut(a, cols)
        assert got.shape == want.shape
        assert np.array_equal(got, want), (cols, kind)


@pytest.mark.parametrize("cols", [1, 160, 161, 320, 2560, 3072, 4096, 13312, 23040])
def test_pattern_grid_is_exact(torch_dev, oracle, cols):
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    print(f"[lut grid] cols={cols}", flush=True)
    rng = np.random.default_rng(cols + 11)
    rows = 64
    for wk in ("random", "plus", "minus", "zero"):
        t = {"random": lambda: rng.integers(-1, 2, size=(rows, cols), dtype=np.int8),
             "plus": lambda: np.ones((rows, cols), np.int8),
             "minus": lambda: -np.ones((rows, cols), np.int8),
             "zero": lambda: np.zeros((rows, cols), np.int8)}[wk]()
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
        for ak in ("random", "max", "min", "alternating"):
            a = acts_of(ak, cols, rng)
            lut = gpu_lut(torch, a, cols)
            out = torch.empty(rows, dtype=torch.int32, device="cuda")
            layer.gemv_lut_i32(lut, out)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().astype(np.int64), exact_gemv(t, a)), (cols, wk, ak)
        layer.close()


@pytest.mark.parametrize("rows,cols", [(1, 160), (65, 161), (130, 3072), (2560, 2560), (1024, 3072), (3072, 23040),
                                       (23040, 3072), (7, 131072)])
def test_shapes_repeat_and_match_the_digit_gemv(torch_dev, oracle, rows, cols):
    """Exact at model and awkward shapes, the same after repeated calls (the atomic slice sums are cleared by the last
    slice of each tile group), and the fp32 outputs equal the digit-table GEMV's bit for bit."""
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    print(f"[lut shapes] {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 0.03)
    want = exact_gemv(t, a)
    da = torch.from_numpy(a).cuda()
    lut = gpu_lut(torch, a, cols)
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    for _ in range(3):
        out.fill_(-1)
        layer.gemv_lut_i32(lut, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().astype(np.int64), want)
    yl = torch.empty(rows, dtype=torch.float32, device="cuda")
    yd = torch.empty(rows, dtype=torch.float32, device="cuda")
    for s in (1.0, 0.37, 0.0, float("nan")):
        layer.gemv_lut_f32(lut, s, yl)
        layer.gemv_f32(da, s, yd)
        torch.cuda.synchronize()
        assert np.array_equal(yl.cpu().numpy().view(np.uint32), yd.cpu().numpy().view(np.uint32)), s
    layer.close()


def test_config0_exact(torch_dev, oracle):
    """BASELINE.json config 0 through the tables: W 2560x2560, P(-1)=P(+1)=0.35, x uniform in [-127, 127]."""
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    t = oracle.gen_trits(0xC0FFEE, (2560, 2560))
    a = oracle.gen_i8(0xBEEF, 2560, -127, 127)
    planar = oracle.pack_matrix(t)
    layer = VelurexHipLayer(planar, 2560, 2560, 0.02)
    out = torch.empty(2560, dtype=torch.int32, device="cuda")
    layer.gemv_lut_i32(gpu_lut(torch, a, 2560), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oracle.gemv_lut_planar(planar, 2560, 2560, a))
    layer.close()


def test_table_plan_equals_the_digit_plan(torch_dev, oracle):
    """vx_lut_plan_create: mixed shapes, int32 and fp32 (device scales), split K slices, run twice with new inputs;
    every output equals the digit-table plan's on the same activations, bit for bit."""
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    rng = np.random.default_rng(4242)
    shapes = [(5120, 3072), (3072, 3072), (3072, 23040), (65, 161), (1, 1), (1100, 160), (7, 131072), (2560, 6912)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    layers, mats, staged, luts, outs_d, outs_l, scales, jd, jl = [], [], [], [], [], [], [], [], []
    for i, (rows, cols) in enumerate(shapes):
        print(f"[lut plan] job {i}: {rows}x{cols}", flush=True)
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, float(0.01 * (i + 1)))
        nb = _lib.staged_bytes(cols)
        st = torch.empty(nb, dtype=torch.uint8, device="cuda")
        lb = _lib.compact_lut_bytes(cols)
        lt = torch.empty(lb, dtype=torch.int8, device="cuda")
        f32 = i % 2 == 1
        dt = torch.float32 if f32 else torch.int32
        od, ol = torch.empty(rows, dtype=dt, device="cuda"), torch.empty(rows, dtype=dt, device="cuda")
        sc = torch.tensor([0.5 + i], dtype=torch.float32, device="cuda")
        layers.append(layer), mats.append(t), staged.append(st), luts.append(lt)
        outs_d.append(od), outs_l.append(ol), scales.append(sc)
        jd.append(_lib.GemvJob(out_f32=int(f32), matrix=layer.handle.value, staged=st.data_ptr(), staged_len=nb,
                               act_scale_dev=sc.data_ptr(), out=od.data_ptr(), out_capacity=rows))
        jl.append(_lib.GemvJob(out_f32=int(f32), matrix=layer.handle.value, staged=lt.data_ptr(), staged_len=lb,
                               act_scale_dev=sc.data_ptr(), out=ol.data_ptr(), out_capacity=rows))
    plan_d, plan_l = _lib.Plan(jd), _lib.LutPlan(jl)
    assert plan_l.work_items() > 0
    for rep in range(2):
        acts = []
        for (rows, cols), st, lt in zip(shapes, staged, luts):
            a = rng.integers(-128, 128, size=cols, dtype=np.int8)
            da = torch.from_numpy(a).cuda()
            _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(da.data_ptr()), cols, cols, ctypes.c_void_p(st.data_ptr()),
                                           st.numel(), stream))
            _lib.compact_lut_dev(da.data_ptr(), cols, cols, lt.data_ptr(), lt.numel(), stream)
            acts.append(a)
        for o in outs_l:
            o.fill_(-1)
        plan_d.run(stream)
        plan_l.run(stream)
        torch.cuda.synchronize()
        for i, ((rows, cols), t, a, od, ol) in enumerate(zip(shapes, mats, acts, outs_d, outs_l)):
            gd, gl = od.cpu().numpy(), ol.cpu().numpy()
            assert np.array_equal(gd.view(np.uint32), gl.view(np.uint32)), (rep, i)
            if i % 2 == 0:
                assert np.array_equal(gl.astype(np.int64), exact_gemv(t, a)), (rep, i)
    plan_d.close(), plan_l.close()
    for layer in layers:
        layer.close()


def test_table_errors(torch_dev, oracle):
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    t = np.ones((64, 320), np.int8)
    layer = VelurexHipLayer(oracle.pack_matrix(t), 64, 320, 1.0)
    lb = _lib.compact_lut_bytes(320)
    assert lb == 2 * 64 * 64
    lut = torch.zeros(lb + 16, dtype=torch.int8, device="cuda")
    out = torch.empty(64, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    short = L.vx_gemv_lut_i32_dev(layer.handle, ctypes.c_void_p(lut.data_ptr()), lb - 1, ctypes.c_void_p(out.data_ptr()),
                                  64, st)
    assert short == 4  # VX_ERR_BUFFER_TOO_SMALL
    misaligned = L.vx_gemv_lut_i32_dev(layer.handle, ctypes.c_void_p(lut.data_ptr() + 1), lb,
                                       ctypes.c_void_p(out.data_ptr()), 64, st)
    assert misaligned == 2  # VX_ERR_INVALID_ARGUMENT
    layer.close()
