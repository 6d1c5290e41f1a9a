"""GPU parity of the block-scaled (Q2_0 x Q8_0) GEMV through the C ABI.

The reference's definition is dot_row_scalar (quintrit-core/src/block_scaled.rs:175-202), restated by the oracle
(vxo_q2_0_dot_row). The GPU keeps its fp32 order, so outputs are compared bit for bit; the config's own bounds (int32
lane sums exact, fp32 within 1e-6 relative) are asserted as well. Weight scales are fp16 (one per 64 weights, stored
beside the trits), widened exactly to the f32 the reference uses; activation scales are f32, one per 32 values.
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


def log_uniform(rng, n, lo=0.005, hi=0.05):
    return np.exp(rng.uniform(np.log(lo), np.log(hi), size=n))


def make_case(oracle, rng, rows, cols):
    t = oracle.gen_trits(int(rng.integers(1 << 30)), (rows, cols))
    ws16 = log_uniform(rng, rows * cols // 64).astype(np.float16)
    acts = oracle.gen_i8(int(rng.integers(1 << 30)), cols, -127, 127)
    as32 = log_uniform(rng, cols // 32).astype(np.float32)
    return t, ws16, acts, as32


def run_q2(torch, mat, acts, as32):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = torch.from_numpy(acts).cuda()
    s = torch.from_numpy(as32).cuda()
    out = torch.full((mat.rows,), float("nan"), dtype=torch.float32, device="cuda")
    mat.gemv_f32(a, s, out, stream)
    lanes = torch.empty(mat.rows * (mat.cols // 32) * 8, dtype=torch.int32, device="cuda")
    mat.lane_sums(a, lanes, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy(), lanes.cpu().numpy().reshape(mat.rows, mat.cols // 32, 8)


@pytest.mark.parametrize("rows,cols", [(1, 64), (7, 128), (8, 192), (9, 640), (65, 704), (130, 4096), (1000, 1600),
                                       (129, 12288), (2049, 320),
                                       (66000, 64)])  # more items than two workgroups per CU: the 16-wave instance
def test_q2_bit_exact_vs_oracle(torch_dev, oracle, rows, cols):
    from quintrit_amd import _lib
    print(f"[q2] {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 1000 + cols)
    t, ws16, acts, as32 = make_case(oracle, rng, rows, cols)
    planar = oracle.pack_matrix(t)
    mat = _lib.Q2Matrix(planar, ws16, rows, cols)
    got, lanes = run_q2(torch_dev, mat, acts, as32)
    want = oracle.q2_0_gemv(planar, ws16.astype(np.float32), acts, as32, rows, cols)
    assert np.array_equal(lanes, oracle.q2_0_lane_sums(planar, acts, rows, cols))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    mat.close()


def test_q2_config4_shapes_and_plan(torch_dev, oracle):
    """The Qwen3-8B-like projections of configs[4] (hidden 4096, FFN 12288, q/o 4096x4096, k/v 1024x4096), one plan."""
    from quintrit_amd import _lib
    torch = torch_dev
    rng = np.random.default_rng(4)
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]
    mats, cases, jobs, outs, keep = [], [], [], [], []
    for rows, cols in shapes:
        t, ws16, acts, as32 = make_case(oracle, rng, rows, cols)
        planar = oracle.pack_matrix(t)
        m = _lib.Q2Matrix(planar, ws16, rows, cols)
        a, s = torch.from_numpy(acts).cuda(), torch.from_numpy(as32).cuda()
        out = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        jobs.append(_lib.Q2Job(matrix=m.handle.value, acts=a.data_ptr(), acts_len=cols, act_scales=s.data_ptr(),
                               n_act_scales=cols // 32, out=out.data_ptr(), out_capacity=rows))
        mats.append(m), cases.append((planar, ws16, acts, as32)), outs.append(out), keep.append((a, s))
    plan = _lib.Q2Plan(jobs)
    plan.run(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for (rows, cols), (planar, ws16, acts, as32), out, m in zip(shapes, cases, outs, mats):
        print(f"[q2 config4] {rows}x{cols}", flush=True)
        got = out.cpu().numpy()
        want = oracle.q2_0_gemv(planar, ws16.astype(np.float32), acts, as32, rows, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # the config's stated bound, on the same numbers
        assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want))
        m.close()
    plan.close()


def test_q2_plan_many_ragged_jobs(torch_dev, oracle):
    """A plan with more items than CUs and items of very different lengths: 300 jobs of ragged shapes (partial tiles
    and tile groups, 1 to 77 blocks per row) around one 4096 x 12288 projection. The plan hands each workgroup a
    balanced list of items; every output must be written exactly as the oracle computes it (outputs start as NaN, so an
    item left out shows)."""
    from quintrit_amd import _lib
    torch = torch_dev
    rng = np.random.default_rng(44)
    shapes = [(int(rng.integers(1, 700)), int(rng.choice([64, 128, 320, 640, 1600, 3200]))) for _ in range(150)]
    shapes += [(4096, 12288)]
    shapes += [(int(rng.integers(1, 1200)), int(rng.choice([64, 704, 4096]))) for _ in range(150)]
    mats, cases, jobs, outs, keep = [], [], [], [], []
    for rows, cols in shapes:
        t, ws16, acts, as32 = make_case(oracle, rng, rows, cols)
        planar = oracle.pack_matrix(t)
        m = _lib.Q2Matrix(planar, ws16, rows, cols)
        a, s = torch.from_numpy(acts).cuda(), torch.from_numpy(as32).cuda()
        out = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        jobs.append(_lib.Q2Job(matrix=m.handle.value, acts=a.data_ptr(), acts_len=cols, act_scales=s.data_ptr(),
                               n_act_scales=cols // 32, out=out.data_ptr(), out_capacity=rows))
        mats.append(m), cases.append((planar, ws16, acts, as32)), outs.append(out), keep.append((a, s))
    wants = [oracle.q2_0_gemv(planar, ws16.astype(np.float32), acts, as32, rows, cols)
             for (rows, cols), (planar, ws16, acts, as32) in zip(shapes, cases)]
    plan = _lib.Q2Plan(jobs)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for run in range(2):
        print(f"[q2 ragged plan] run {run}", flush=True)
        plan.run(stream)
        torch.cuda.synchronize()
        for i, ((rows, cols), out, want) in enumerate(zip(shapes, outs, wants)):
            got = out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (i, rows, cols)
            out.fill_(float("nan"))
    plan.close()
    for m in mats:
        m.close()
