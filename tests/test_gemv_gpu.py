"""GPU parity of the velurex GEMV (libvelurex_hip through its C ABI) against the oracle and brute force.

The integer results must be bit-exact; the fp32 epilogue must equal the oracle's bit for bit (it is one fp32 division
and one fp32 multiplication per row, layer.rs:246-253). Shapes and patterns follow the reference's GPU tests
(quintrit-cuda/tests/gemv.rs:46-64,77-125) and BASELINE.json configs 0-2.
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


def weights(kind, rows, cols, rng):
    return {"random": lambda: rng.integers(-1, 2, size=(rows, cols), dtype=np.int8),
            "plus": lambda: np.ones((rows, cols), np.int8),
            "minus": lambda: -np.ones((rows, cols), np.int8),
            "zero": lambda: np.zeros((rows, cols), np.int8)}[kind]()


def activations(kind, cols, rng):
    return {"random": lambda: rng.integers(-128, 128, size=cols, dtype=np.int8),
            "max": lambda: np.full(cols, 127, np.int8),
            "min": lambda: np.full(cols, -128, np.int8),
            "alternating": lambda: np.where(np.arange(cols) % 2 == 0, 127, -128).astype(np.int8)}[kind]()


def gpu_gemv_i32(torch, layer, acts):
    a = torch.from_numpy(acts).cuda()
    out = torch.empty(layer.shape()[0], dtype=torch.int32, device="cuda")
    layer.gemv_i32(a, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("cols", [1, 160, 161, 320, 2560, 3072, 4096, 13312, 23040])
def test_pattern_grid_is_exact(torch_dev, oracle, cols):
    from quintrit_amd import VelurexHipLayer
    print(f"[gemv grid] cols={cols}", flush=True)
    rng = np.random.default_rng(cols)
    rows = 64
    for wk in ("random", "plus", "minus", "zero"):
        t = weights(wk, rows, cols, rng)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
        for ak in ("random", "max", "min", "alternating"):
            a = activations(ak, cols, rng)
            got = gpu_gemv_i32(torch_dev, layer, a)
            assert np.array_equal(got.astype(np.int64), exact_gemv(t, a)), (cols, wk, ak)
        layer.close()


@pytest.mark.parametrize("rows,cols", [(1, 160), (2, 160), (6, 3072), (12, 2560), (40, 3072), (65, 161),
                                       (2560, 2560), (3456, 2560), (1024, 3072), (3072, 23040), (23040, 3072),
                                       (5120, 3072), (7, 131072)])
def test_awkward_and_model_shapes(torch_dev, oracle, rows, cols):
    from quintrit_amd import VelurexHipLayer
    print(f"[gemv shapes] {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 131 + cols)
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    want = exact_gemv(t, a)
    for _ in range(3):  # the split-K accumulators must be clean again after every call
        got = gpu_gemv_i32(torch_dev, layer, a)
        assert np.array_equal(got.astype(np.int64), want)
    layer.close()


def test_config0_exact_and_epilogue(torch_dev, oracle):
    """W 2560x2560, P(-1)=P(+1)=0.35, x uniform in [-127, 127], y = float(acc) * 0.02."""
    from quintrit_amd import VelurexHipLayer
    t = oracle.gen_trits(0xC0FFEE, (2560, 2560))
    a = oracle.gen_i8(0xBEEF, 2560, -127, 127)
    planar = oracle.pack_matrix(t)
    layer = VelurexHipLayer(planar, 2560, 2560, 0.02)
    acc = gpu_gemv_i32(torch_dev, layer, a)
    want = oracle.gemv_lut_planar(planar, 2560, 2560, a)
    assert np.array_equal(acc, want)
    assert np.array_equal(acc.astype(np.int64), oracle.gemv_bruteforce(t, a))
    y = np.empty(2560, np.float32)
    layer.forward(a, 1.0, y)                       # TernaryGemvLayer::forward with act_scale = 1
    assert np.array_equal(y.view(np.uint32), oracle.epilogue_f32(want, 0.02, 1.0).view(np.uint32))
    layer.forward(a, 0.37, y)
    assert np.array_equal(y.view(np.uint32), oracle.epilogue_f32(want, 0.02, 0.37).view(np.uint32))
    for bad in (0.0, -1.0, float("nan")):
        layer.forward(a, bad, y)
        assert np.array_equal(y.view(np.uint32), np.zeros(2560, np.uint32))   # +0.0, as out.fill(0.0)
    layer.close()


@pytest.mark.parametrize("rows,cols", [(1, 5), (64, 160), (70, 777), (1024, 3072), (3072, 3072), (2100, 23040)])
def test_layer_forward_calls_in_a_row(torch_dev, oracle, rows, cols):
    """vx_layer_forward (the caller waits on the GEMV's completion flag in its pinned buffer) over shapes with one K
    slice and with split slices in one or several tile groups: eight calls in a row with new activations and scales,
    each equal to the oracle's epilogue bit for bit, interleaved with vx_gemv_f32_dev on device buffers of the same
    matrix (which shares its slice sums and tickets), and a call with a zero scale between them."""
    from quintrit_amd import VelurexHipLayer
    torch = torch_dev
    print(f"[layer_forward] {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    planar = oracle.pack_matrix(t)
    layer = VelurexHipLayer(planar, rows, cols, 0.05)
    y = np.empty(rows, np.float32)
    for call in range(8):
        a = activations(("random", "max", "min", "alternating")[call % 4], cols, rng)
        sc = float(rng.uniform(0.1, 3.0))
        want = exact_gemv(t, a).astype(np.int32)
        layer.forward(a, sc, y)
        assert np.array_equal(y.view(np.uint32), oracle.epilogue_f32(want, 0.05, sc).view(np.uint32)), call
        if call % 3 == 1:
            yd = torch.empty(rows, dtype=torch.float32, device="cuda")
            layer.gemv_f32(torch.from_numpy(a).cuda(), sc, yd)
            torch.cuda.synchronize()
            assert np.array_equal(yd.cpu().numpy().view(np.uint32), y.view(np.uint32)), call
        if call == 4:
            layer.forward(a, 0.0, y)
            assert np.array_equal(y.view(np.uint32), np.zeros(rows, np.uint32))
    layer.close()


def test_staged_activations_shared_by_matrices(torch_dev, oracle):
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    rng = np.random.default_rng(99)
    cols = 3072
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    da = torch.from_numpy(a).cuda()
    nbytes = _lib.staged_bytes(cols)
    staged = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    L = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(da.data_ptr()), cols, cols, ctypes.c_void_p(staged.data_ptr()),
                                   nbytes, stream))
    for rows in (3072, 1024, 23040):
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 0.05)
        out = torch.empty(rows, dtype=torch.int32, device="cuda")
        _lib.check(L.vx_gemv_staged_i32_dev(layer.handle, ctypes.c_void_p(staged.data_ptr()), nbytes,
                                            ctypes.c_void_p(out.data_ptr()), rows, stream))
        outf = torch.empty(rows, dtype=torch.float32, device="cuda")
        _lib.check(L.vx_gemv_staged_f32_dev(layer.handle, ctypes.c_void_p(staged.data_ptr()), nbytes,
                                            ctypes.c_float(0.25), ctypes.c_void_p(outf.data_ptr()), rows, stream))
        torch.cuda.synchronize()
        want = exact_gemv(t, a)
        assert np.array_equal(out.cpu().numpy().astype(np.int64), want)
        assert np.array_equal(outf.cpu().numpy().view(np.uint32),
                              oracle.epilogue_f32(want.astype(np.int32), 0.05, 0.25).view(np.uint32))
        layer.close()


def test_create_from_device_memory(torch_dev, oracle):
    from quintrit_amd import _lib
    torch = torch_dev
    L = _lib.lib()
    for rows, cols in ((100, 3072), (64, 161), (3, 23040)):
        rng = np.random.default_rng(rows + cols)
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        planar = oracle.pack_matrix(t)
        dp = torch.from_numpy(planar.reshape(-1)).cuda()
        h = ctypes.c_void_p()
        _lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(dp.data_ptr()), planar.size, rows, cols, ctypes.c_float(1.0),
                                          ctypes.byref(h)))
        # the device transform writes exactly the host layout
        wp = ctypes.c_void_p()
        _lib.check(L.vx_matrix_device_weights(h, ctypes.byref(wp)))
        n = _lib.layout(rows, cols)["device_bytes"]
        host = np.empty(n, np.uint8)
        torch.cuda.synchronize()
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        assert hip.hipMemcpy(host.ctypes.data_as(ctypes.c_void_p), wp, n, 2) == 0
        assert np.array_equal(host, _lib.device_layout_pack(planar, rows, cols))
        a = rng.integers(-128, 128, size=cols, dtype=np.int8)
        da = torch.from_numpy(a).cuda()
        out = torch.empty(rows, dtype=torch.int32, device="cuda")
        _lib.check(L.vx_gemv_i32_dev(h, ctypes.c_void_p(da.data_ptr()), cols, ctypes.c_void_p(out.data_ptr()), rows,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().astype(np.int64), exact_gemv(t, a))
        _lib.check(L.vx_matrix_free(h))
    # an invalid byte in device memory is reported with its index
    planar = oracle.pack_matrix(np.zeros((2, 160), np.int8))
    planar[1, 3] = 252
    dp = torch.from_numpy(planar.reshape(-1)).cuda()
    h = ctypes.c_void_p()
    st = L.vx_matrix_create_dev(ctypes.c_void_p(dp.data_ptr()), planar.size, 2, 160, ctypes.c_float(1.0), ctypes.byref(h))
    assert st == 5 and b"byte 35" in L.vx_last_error_message()


def test_planar_oneshot_api(torch_dev, oracle):
    from quintrit_amd import gemv_planar_f32, gemv_planar_i32
    rng = np.random.default_rng(5)
    t = rng.integers(-1, 2, size=(96, 3072), dtype=np.int8)
    a = rng.integers(-128, 128, size=3072, dtype=np.int8)
    planar = oracle.pack_matrix(t)
    got = gemv_planar_i32(planar, 96, 3072, a)
    assert np.array_equal(got.astype(np.int64), exact_gemv(t, a))
    f = gemv_planar_f32(planar, 96, 3072, a, 0.125)
    assert np.array_equal(f.view(np.uint32), oracle.scale_f32(got, 0.125).view(np.uint32))


# The reference's kernel-level C API tests (quintrit-c/tests/ffi_kernel.rs:36-49,195-228): full tiles, remainder rows
# and columns, partial 160-trit blocks, degenerate sizes, and three realistic projections.
FFI_SHAPES = [(1, 1), (3, 5), (5, 7), (32, 160), (33, 161), (31, 159), (64, 320), (65, 250), (96, 3072), (100, 1000),
              (130, 640), (192, 33), (512, 3072), (96, 6000), (70, 777)]


@pytest.mark.parametrize("rows,cols", FFI_SHAPES)
def test_planar_oneshot_reference_ffi_shapes(torch_dev, oracle, rows, cols):
    """vx_gemv_planar_i32 / _f32 (the argument order of quintrit_gemv_i32 / _f32) against the brute-force int64
    product, and out = float(acc) * 0.25 bit for bit, as check_gemv asserts (ffi_kernel.rs:195-222)."""
    from quintrit_amd import gemv_planar_f32, gemv_planar_i32
    print(f"[gemv ffi] {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 131 + cols)
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    planar = oracle.pack_matrix(t)
    want = t.astype(np.int64) @ a.astype(np.int64)
    got = gemv_planar_i32(planar, rows, cols, a)
    assert np.array_equal(got.astype(np.int64), want)
    f = gemv_planar_f32(planar, rows, cols, a, 0.25)
    assert np.array_equal(f.view(np.uint32), (want.astype(np.float32) * np.float32(0.25)).view(np.uint32))


def test_planar_oneshot_extreme_activations(torch_dev, oracle):
    """All weights +1 or -1 against constant activations -128, 127, 0, -1, 1 at 64 x 1000: every output is
    w * fill * cols, the largest sums a row reaches (ffi_kernel.rs:225-248)."""
    from quintrit_amd import gemv_planar_i32
    rows, cols = 64, 1000
    for fill in (-128, 127, 0, -1, 1):
        for w in (1, -1):
            planar = oracle.pack_matrix(np.full((rows, cols), w, np.int8))
            got = gemv_planar_i32(planar, rows, cols, np.full(cols, fill, np.int8))
            assert np.all(got == w * fill * cols), (fill, w)


def test_golden_fixtures(torch_dev):
    """The committed fixtures (tests/golden) reproduce on the GPU."""
    import os
    from quintrit_amd import VelurexHipLayer
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    for name in sorted(os.listdir(gdir)):
        if not (name.startswith("gemv_") and name.endswith(".npz")):
            continue
        z = np.load(os.path.join(gdir, name))
        rows, cols = (int(v) for v in z["shape"])
        layer = VelurexHipLayer(z["planar"], rows, cols, float(z["weight_scale"]))
        acc = gpu_gemv_i32(torch_dev, layer, z["acts"])
        assert np.array_equal(acc, z["acc"]), name
        y = np.empty(rows, np.float32)
        layer.forward(z["acts"], float(z["act_scale"]), y)
        assert np.array_equal(y.view(np.uint32), z["y"].view(np.uint32)), name
        layer.close()


def test_plan_stages_raw_activations(torch_dev, oracle):
    """Jobs that bring raw int8 activations (vx_gemv_job_t.acts): each run stages every distinct (acts, staged) pair
    in one launch, then runs the GEMVs. Two jobs share one input (as q/k/v do), one job reads an input the caller
    staged, one gives no acts field at all (the smaller struct_size); all outputs equal brute force, on two runs with
    new activations; a staged buffer claimed by two different inputs is refused."""
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    rng = np.random.default_rng(77)
    shapes = [(1024, 3072), (1024, 3072), (3072, 23040), (65, 161), (130, 3072)]
    share = {0: 0, 1: 0, 2: 1, 3: 2, 4: 3}  # job -> input
    cols_of = {0: 3072, 1: 23040, 2: 161, 3: 3072}
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    raw = {k: torch.empty(c, dtype=torch.int8, device="cuda") for k, c in cols_of.items()}
    staged = {k: torch.empty(_lib.staged_bytes(c), dtype=torch.uint8, device="cuda") for k, c in cols_of.items()}
    layers, mats, outs, jobs = [], [], [], []
    for i, (rows, cols) in enumerate(shapes):
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
        out = torch.empty(rows, dtype=torch.int32, device="cuda")
        k = share[i]
        j = _lib.GemvJob(out_f32=0, matrix=layer.handle.value, staged=staged[k].data_ptr(),
                         staged_len=staged[k].numel(), out=out.data_ptr(), out_capacity=rows,
                         acts=None if k == 3 else raw[k].data_ptr())
        if k == 3:
            j.struct_size = _lib.GemvJob.acts.offset  # a caller built against the job without the acts field
        layers.append(layer), mats.append(t), outs.append(out), jobs.append(j)
    plan = _lib.Plan(jobs)
    for rep in range(2):
        acts = {k: rng.integers(-128, 128, size=c, dtype=np.int8) for k, c in cols_of.items()}
        for k, a in acts.items():
            raw[k].copy_(torch.from_numpy(a))
        # input 3 is the caller's own staging (no acts in its job)
        _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(raw[3].data_ptr()), 3072, 3072,
                                       ctypes.c_void_p(staged[3].data_ptr()), staged[3].numel(), stream))
        plan.run(stream)
        torch.cuda.synchronize()
        for i, (t, out) in enumerate(zip(mats, outs)):
            assert np.array_equal(out.cpu().numpy().astype(np.int64), exact_gemv(t, acts[share[i]])), (rep, i)
    plan.close()
    bad = [_lib.GemvJob(out_f32=0, matrix=layers[0].handle.value, staged=staged[0].data_ptr(),
                        staged_len=staged[0].numel(), out=outs[0].data_ptr(), out_capacity=1024,
                        acts=raw[0].data_ptr()),
           _lib.GemvJob(out_f32=0, matrix=layers[1].handle.value, staged=staged[0].data_ptr(),
                        staged_len=staged[0].numel(), out=outs[1].data_ptr(), out_capacity=1024,
                        acts=raw[3].data_ptr())]
    with pytest.raises(_lib.VxError, match="INVALID_ARGUMENT"):
        _lib.Plan(bad)
    for layer in layers:
        layer.close()


def test_batched_plan_mixed_jobs(torch_dev, oracle):
    """vx_plan_*: many GEMVs in one persistent launch, int32 and fp32 (scale read from device memory), long rows split
    into K slices; the plan runs again after its inputs change (its pointers are fixed, the contents are not)."""
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    rng = np.random.default_rng(2024)
    shapes = [(5120, 3072), (3072, 3072), (3072, 23040), (65, 161), (1, 1), (1100, 160), (7, 131072), (2560, 6912)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    layers, mats, staged, outs, scales, jobs = [], [], [], [], [], []
    for i, (rows, cols) in enumerate(shapes):
        print(f"[plan] job {i}: {rows}x{cols}", flush=True)
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, float(0.01 * (i + 1)))
        nb = _lib.staged_bytes(cols)
        st = torch.empty(nb, dtype=torch.uint8, device="cuda")
        f32 = i % 2 == 1
        out = torch.empty(rows, dtype=torch.float32 if f32 else torch.int32, device="cuda")
        sc = torch.tensor([0.5 + i], dtype=torch.float32, device="cuda")
        layers.append(layer), mats.append(t), staged.append(st), outs.append(out), scales.append(sc)
        jobs.append(_lib.GemvJob(out_f32=int(f32), matrix=layer.handle.value, staged=st.data_ptr(), staged_len=nb,
                                 act_scale_dev=sc.data_ptr(), out=out.data_ptr(), out_capacity=rows))
    plan = _lib.Plan(jobs)
    assert plan.work_items() > 0
    for rep in range(2):
        acts = []
        for (rows, cols), st in zip(shapes, staged):
            a = rng.integers(-128, 128, size=cols, dtype=np.int8)
            da = torch.from_numpy(a).cuda()
            _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(da.data_ptr()), cols, cols, ctypes.c_void_p(st.data_ptr()),
                                           st.numel(), stream))
            acts.append(a)
        plan.run(stream)
        torch.cuda.synchronize()
        for i, ((rows, cols), t, a, out) in enumerate(zip(shapes, mats, acts, outs)):
            want = exact_gemv(t, a)
            got = out.cpu().numpy()
            if i % 2 == 1:
                y = oracle.epilogue_f32(want.astype(np.int32), float(np.float32(0.01 * (i + 1))), 0.5 + i)
                assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), (rep, i)
            else:
                assert np.array_equal(got.astype(np.int64), want), (rep, i)
    # a non-positive device scale gives zeros (layer.rs:246-253)
    scales[1].fill_(0.0)
    plan.run(stream)
    torch.cuda.synchronize()
    assert np.array_equal(outs[1].cpu().numpy().view(np.uint32), np.zeros(shapes[1][0], np.uint32))
    plan.close()
    for layer in layers:
        layer.close()


def test_plan_in_hip_graph_replays(torch_dev, oracle):
    """A plan captured in a HIP graph gives the eager result on every replay, with eager work in between."""
    from quintrit_amd import VelurexHipLayer, _lib
    torch = torch_dev
    L = _lib.lib()
    rng = np.random.default_rng(77)
    rows, cols = 3072, 23040
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    layer = VelurexHipLayer(oracle.pack_matrix(t), rows, cols, 1.0)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    da = torch.from_numpy(a).cuda()
    nb = _lib.staged_bytes(cols)
    st = torch.empty(nb, dtype=torch.uint8, device="cuda")
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    plan = _lib.Plan([_lib.GemvJob(out_f32=0, matrix=layer.handle.value, staged=st.data_ptr(), staged_len=nb,
                                   act_scale_dev=None, out=out.data_ptr(), out_capacity=rows)])
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        sp = ctypes.c_void_p(s.cuda_stream)
        _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(da.data_ptr()), cols, cols, ctypes.c_void_p(st.data_ptr()), nb, sp))
        plan.run(sp)
    torch.cuda.synchronize()
    eager = out.cpu().numpy().copy()
    assert np.array_equal(eager.astype(np.int64), exact_gemv(t, a))
    with torch.cuda.graph(g, stream=s):
        sp = ctypes.c_void_p(s.cuda_stream)
        _lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(da.data_ptr()), cols, cols, ctypes.c_void_p(st.data_ptr()), nb, sp))
        plan.run(sp)
    for _ in range(4):
        out.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager)
    plan.close()
    layer.close()
