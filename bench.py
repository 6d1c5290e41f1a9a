#!/usr/bin/env python3
"""Velurex ternary GEMV decode weight stream on one MI355X.

One "step" is the projection stream of one decoded Falcon3-10B token at bs=1: for each of the 40 layers the stacked
q|k|v projection (5120 x 3072), o (3072 x 3072), the row-interleaved gate|up projection (46080 x 3072) and down
(3072 x 23040) -- 9,500,098,560 ternary weights, 1.90 GB at 1.60 bpw -- each on its own int8 input vector (per-token
absmax int8 of N(0,1) fp32), with the fp32 epilogue. The reference measures the same projection set as CUDA graphs
(docs/benchmarks.md, "Projections against Microsoft's W2A8 GPU kernel"); here they are one batched plan (vx_plan_run:
one persistent GEMV launch plus the K-slice finish), and, for comparison, 160 lone-GEMV launches in one HIP graph.
Weights are i.i.d. trits, P(-1) = P(+1) = 0.35, generated on the GPU, far larger than the 256 MB last-level cache,
so every replay streams them from HBM. Inputs are resident in HBM when the timed region starts.

Prints one JSON line (the driver's contract). `--gpus N` with N > 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Gweights/s + HBM GB/s (% of peak), Falcon3-10B decode GEMV; tok/s at bs=1"
HBM_PEAK_GBPS = 8000.0
LAYERS, HIDDEN, FFN, KV = 40, 3072, 23040, 1024
# (name, rows, cols): the launches of one layer; q|k|v stacked, gate|up interleaved row by row.
LAYER_SHAPES = [("qkv", HIDDEN + 2 * KV, HIDDEN), ("o", HIDDEN, HIDDEN), ("gate_up", 2 * FFN, HIDDEN),
                ("down", HIDDEN, FFN)]
REF_CPU_GWEIGHTS = 221.6  # quintrit_512, 4 threads, EPYC 9V45 (docs/benchmarks.md:77)
# HBM bytes of one full-step gemv_kernel launch, from rocprofv3 FETCH_SIZE and WRITE_SIZE scaled by a plain-copy
# calibration (profiles/gemv_kernel_falcon3_projection_stream.md). Only valid for the default 40-layer workload.
TRAFFIC_BYTES_PER_STEP = 1_893_508 * 1024


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=LAYERS, help=argparse.SUPPRESS)  # smoke runs only
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--workload", choices=["stream", "gemm", "q2"], default="stream",
                    help="stream: the driver's line (configs[1]); gemm: the batched GEMM of configs[2]; q2: the "
                         "block-scaled GEMV stream of configs[4]")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB device to device 5 times (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def random_planar(torch, rows: int, cols: int, gen) -> "torch.Tensor":
    """Planar velurex bytes (quintrit-core/src/pack.rs:66-131) of i.i.d. trits with P(-1)=P(+1)=0.35, on the GPU."""
    nb = (cols + 159) // 160
    out = torch.empty(rows * nb * 32, dtype=torch.uint8, device="cuda")
    radix = torch.tensor([1, 3, 9, 28, 84], dtype=torch.int16, device="cuda").view(1, 1, 5, 1)
    step = max(1, (1 << 26) // (nb * 160))
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        u = torch.randint(0, 100, (r1 - r0, nb * 160), dtype=torch.int16, device="cuda", generator=gen)
        d = (u >= 35).to(torch.int16) + (u >= 65).to(torch.int16)  # digit = trit + 1
        if nb * 160 > cols:
            d[:, cols:] = 1  # padding trits are zero
        b = (d.view(r1 - r0, nb, 5, 32) * radix).sum(dim=2).to(torch.uint8)
        out[r0 * nb * 32:r1 * nb * 32] = b.view(-1)
    return out


def quantize_i8(torch, x):
    """Per-token absmax int8 (quintrit-runtime/src/ops.rs:241-267): s = 127/amax, q = round-half-away(x s)."""
    amax = x.abs().max()
    s = 127.0 / amax
    v = x * s
    q = torch.sign(v) * torch.floor(v.abs() + 0.5)
    return q.clamp(-128, 127).to(torch.int8), float(s)


class Stream:
    """The 40-layer projection stream resident on the GPU, with one staged input vector per projection."""

    def __init__(self, torch, L, lib, layers: int):
        self.torch, self.L, self.lib = torch, L, lib
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0x5EED)
        self.mats = []      # per layer: list of (name, handle, rows, cols)
        self.staged = []    # per launch: (tensor, nbytes)
        self.outs = []
        self.weights = 0
        self.alg_bytes = 0
        self.device_bytes = 0
        n = layers * len(LAYER_SHAPES)
        self.scales = torch.empty(n, dtype=torch.float32, device="cuda")
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        k = 0
        for li in range(layers):
            row = []
            for name, rows, cols in LAYER_SHAPES:
                planar = random_planar(torch, rows, cols, gen)
                h = ctypes.c_void_p()
                lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                                 ctypes.c_float(0.02), ctypes.byref(h)))
                del planar
                x = torch.randn(cols, device="cuda", generator=gen, dtype=torch.float32)
                q, s = quantize_i8(torch, x)
                nbytes = lib.staged_bytes(cols)
                staged = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
                lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(q.data_ptr()), cols, cols,
                                              ctypes.c_void_p(staged.data_ptr()), nbytes, stream))
                self.scales[k] = s
                row.append((name, h, rows, cols))
                self.staged.append((staged, nbytes))
                self.outs.append(torch.empty(rows, dtype=torch.float32, device="cuda"))
                self.weights += rows * cols
                self.alg_bytes += rows * cols / 5.0
                self.device_bytes += lib.layout(rows, cols)["device_bytes"]
                k += 1
            self.mats.append(row)
        torch.cuda.synchronize()

    def jobs(self, which=None):
        """vx_gemv_job_t list in model order (all launch types, or only LAYER_SHAPES[which])."""
        out = []
        k = 0
        for row in self.mats:
            for t, (_, h, rows, _) in enumerate(row):
                if which is None or which == t:
                    staged, nbytes = self.staged[k]
                    out.append(self.lib.GemvJob(out_f32=1, matrix=h.value, staged=staged.data_ptr(), staged_len=nbytes,
                                                act_scale_dev=self.scales.data_ptr() + 4 * k,
                                                out=self.outs[k].data_ptr(), out_capacity=rows))
                k += 1
        return out

    def chain_step(self) -> None:
        """The same projections as 160 dependent launches (one GEMV call each, as a decode step issues them)."""
        st = ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)
        k = 0
        for row in self.mats:
            for _, h, rows, _ in row:
                staged, nbytes = self.staged[k]
                self.lib.check(self.L.vx_gemv_staged_f32_dev(h, ctypes.c_void_p(staged.data_ptr()), nbytes,
                                                             ctypes.c_float(1.0), ctypes.c_void_p(self.outs[k].data_ptr()),
                                                             rows, st))
                k += 1

    def free(self):
        for row in self.mats:
            for _, h, _, _ in row:
                self.lib.check(self.L.vx_matrix_free(h))


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # eager warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_fn(torch, fn, steps: int, warmup: int):
    """Average device time per call of fn (torch events on the current stream, which fn launches on) and wall time."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return t0.elapsed_time(t1) / steps, wall


def cpu_baseline(budget_s: float):
    """The CPU oracle's restatement of the reference's table GEMV (oracle/velurex_oracle.c, avx512.rs:1526-1626
    algorithm, scalar C, one thread) timed on this host over a bounded sample: the seven projections of one Falcon3-10B
    layer in model order, repeated until the budget is used."""
    import numpy as np
    from oracle import oracle
    L = oracle.lib()
    shapes = [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    mats = []
    for i, (r, c) in enumerate(shapes):
        t = oracle.gen_trits(100 + i, (r, c))
        planar = oracle.pack_matrix(t)
        tiles = oracle.tile_rows(planar, r, c)
        a = oracle.gen_i8(200 + i, c, -127, 127)
        mats.append((np.ascontiguousarray(tiles), r, c, a, np.empty(r, np.int32)))
    weights = 0
    t0 = time.perf_counter()
    reps = 0
    while True:
        for tiles, r, c, a, out in mats:
            L.vxo_gemv_lut_tilerows(tiles.ctypes.data_as(ctypes.c_void_p), r, c, a.ctypes.data_as(ctypes.c_void_p),
                                    out.ctypes.data_as(ctypes.c_void_p))
            weights += r * c
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": round(weights / dt / 1e9, 3), "unit": "Gweights/s", "cores": 1, "kind": "port",
            "sample": f"{reps} pass(es) over the 7 projections of one Falcon3-10B layer ({sum(r * c for _, r, c, _, _ in mats)} "
                      f"weights/pass), scalar C restatement of the table kernel, 1 thread, {dt:.1f} s"}


def gemm_bench(torch, L, lib, args) -> int:
    """Y = X W^T for W 23040 x 3072 and 3072 x 23040 (velurex), X M x K int8 quantized per
    token from N(0,1), M in {8, 32, 128, 512}; exact int32 on the matrix cores. One JSON line per call of this mode;
    ops = 2 M N K; bytes = weights (N K / 5) + X + Y."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC2)
    results = []
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rows, cols in ((23040, 3072), (3072, 23040)):
        planar = random_planar(torch, rows, cols, gen)
        h = ctypes.c_void_p()
        lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                         ctypes.c_float(0.02), ctypes.byref(h)))
        del planar
        for m in (8, 32, 128, 512):
            x = torch.randn((m, cols), device="cuda", generator=gen)
            q = torch.empty((m, cols), dtype=torch.int8, device="cuda")
            for i in range(m):
                q[i] = quantize_i8(torch, x[i])[0]
            y = torch.empty((m, rows), dtype=torch.int32, device="cuda")
            n = ctypes.c_size_t()
            lib.check(L.vx_gemm_workspace_bytes(h, m, ctypes.byref(n)))
            ws = torch.empty(n.value, dtype=torch.uint8, device="cuda")
            call = lambda: lib.check(L.vx_gemm_i32_dev(h, ctypes.c_void_p(q.data_ptr()), m, cols,  # noqa: E731
                                                       ctypes.c_void_p(y.data_ptr()), rows,
                                                       ctypes.c_void_p(ws.data_ptr()), n.value, stream))
            ms, _ = time_fn(torch, call, max(5, args.steps), max(2, args.warmup))
            ops = 2.0 * m * rows * cols
            byts = rows * cols / 5.0 + m * cols + 4.0 * m * rows
            r = {"rows": rows, "cols": cols, "m": m, "us": round(ms * 1e3, 2), "TOPS": round(ops / (ms / 1e3) / 1e12, 2),
                 "GBps": round(byts / (ms / 1e3) / 1e9, 1)}
            log(f"gemm {rows}x{cols} m={m}: {r['us']} us, {r['TOPS']} TOPS, {r['GBps']} GB/s")
            results.append(r)
        lib.check(L.vx_matrix_free(h))
    print(json.dumps({"workload": "batched ternary GEMM, BASELINE.json configs[2]", "dtype": "int8 x ternary -> int32",
                      "data": "synthetic", "note": "time per vx_gemm_i32_dev call (activation staging + GEMM + "
                      "K-slice finish), HIP events", "results": results}), flush=True)
    return 0


def q2_bench(torch, L, lib, args) -> int:
    """the projections of one Qwen3-8B-like token (36 layers; q, o 4096 x 4096; k, v
    1024 x 4096; gate, up 12288 x 4096; down 4096 x 12288) as Q2_0 GEMVs: velurex trits plus one fp16 scale per 64
    weights (log-uniform in [0.005, 0.05]) stored beside them, Q8_0 activations (int8 uniform in [-127, 127], one f32
    scale per 32, log-uniform in [0.005, 0.05]). One step = one plan run over all 252 projections."""
    import numpy as np
    layers = 36 if args.layers == LAYERS else args.layers
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC4)
    rng = np.random.default_rng(0xC4)
    mats, jobs, keep = [], [], []
    weights = 0
    dev_bytes = 0
    log(f"building {layers} layers of Q2_0 matrices")
    for _ in range(layers):
        for rows, cols in shapes:
            planar = random_planar(torch, rows, cols, gen).cpu().numpy()
            ws16 = np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=rows * cols // 64)).astype(np.float16)
            m = lib.Q2Matrix(planar, ws16, rows, cols)
            del planar
            acts = torch.randint(-127, 128, (cols,), dtype=torch.int8, device="cuda", generator=gen)
            a_s = torch.from_numpy(np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=cols // 32))
                                   .astype(np.float32)).cuda()
            out = torch.empty(rows, dtype=torch.float32, device="cuda")
            jobs.append(lib.Q2Job(matrix=m.handle.value, acts=acts.data_ptr(), acts_len=cols, act_scales=a_s.data_ptr(),
                                  n_act_scales=cols // 32, out=out.data_ptr(), out_capacity=rows))
            mats.append(m)
            keep.append((acts, a_s, out))
            weights += rows * cols
            n = ctypes.c_size_t()
            lib.check(L.vx_matrix_memory_bytes(m.handle, ctypes.byref(n)))
            dev_bytes += n.value
    plan = lib.Q2Plan(jobs)
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    ms, _ = time_fn(torch, lambda: plan.run(stream()), args.steps, args.warmup)
    alg = weights / 5.0 + 2.0 * weights / 64.0
    r = {"workload": "Q2_0 projection stream, BASELINE.json configs[4]", "layers": layers, "weights": weights,
         "ms_per_step": round(ms, 4), "Gweights_s": round(weights / (ms / 1e3) / 1e9, 1),
         "alg_bytes": int(alg), "alg_GBps": round(alg / (ms / 1e3) / 1e9, 1),
         "device_bytes": dev_bytes, "device_GBps": round(dev_bytes / (ms / 1e3) / 1e9, 1),
         "tok_s_projection_bound": round(1e3 / ms, 1), "data": "synthetic", "dtype": "int8 x ternary, fp32 chains"}
    log(f"q2 stream: {ms:.4f} ms/step, {r['Gweights_s']} Gweights/s, {r['alg_GBps']} GB/s algorithmic")
    print(json.dumps(r), flush=True)
    plan.close()
    for m in mats:
        m.close()
    return 0


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (how the path would shard over "
                                   "several GPUs is described in DESIGN.md, not built)"}))
        return 2
    import torch
    from quintrit_amd import _lib
    L = _lib.lib()
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        return 1
    torch.cuda.set_device(0)
    if args.copy_probe:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel(), "copies": 5}), flush=True)
        return 0
    if args.workload == "gemm":
        return gemm_bench(torch, L, _lib, args)
    if args.workload == "q2":
        return q2_bench(torch, L, _lib, args)
    log(f"building the {args.layers}-layer weight stream on the GPU")
    st = Stream(torch, L, _lib, args.layers)
    log(f"{st.weights} weights, {st.alg_bytes / 1e9:.4f} GB algorithmic, {st.device_bytes / 1e9:.4f} GB device layout")
    plan = _lib.Plan(st.jobs())
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    step = lambda: plan.run(stream())  # noqa: E731
    log(f"plan: {len(st.jobs())} GEMVs, {plan.work_items()} work items; timing")
    ms, wall = time_fn(torch, step, args.steps, args.warmup)
    gw = st.weights / (ms / 1e3) / 1e9
    gbps = st.alg_bytes / (ms / 1e3) / 1e9
    log(f"{ms:.4f} ms/step, {gw:.1f} Gweights/s, {gbps:.1f} GB/s algorithmic ({gbps / HBM_PEAK_GBPS:.1%} of peak), "
        f"wall {wall / args.steps * 1e3:.4f} ms/step")

    breakdown = {}
    chain = None
    if not args.no_breakdown:
        # each launch type alone, over all layers (distinct weights, so no cache reuse)
        for t, (name, rows, cols) in enumerate(LAYER_SHAPES):
            p = _lib.Plan(st.jobs(t))
            mk, _ = time_fn(torch, lambda p=p: p.run(stream()), max(3, args.steps // 2), 2)
            alg = rows * cols / 5.0 * len(st.mats)
            breakdown[name] = {"rows": rows, "cols": cols, "us_per_matrix": round(mk * 1e3 / len(st.mats), 3),
                               "alg_GBps": round(alg / (mk / 1e3) / 1e9, 1)}
            log(f"  {name:8s} {rows}x{cols}: {mk * 1e3 / len(st.mats):.2f} us/matrix, {alg / (mk / 1e3) / 1e9:.1f} GB/s")
            p.close()
        # the dependent form: one GEMV launch per projection, captured as one HIP graph
        g = capture(torch, st.chain_step)
        mc, _ = time_fn(torch, g.replay, max(3, args.steps // 2), 2)
        chain = {"ms_per_step": round(mc, 4), "Gweights_s": round(st.weights / (mc / 1e3) / 1e9, 1),
                 "alg_GBps": round(st.alg_bytes / (mc / 1e3) / 1e9, 1), "launches": len(st.jobs()),
                 "note": "one lone-GEMV call per projection (each waits for the previous), as a HIP graph"}
        log(f"  chain of {len(st.jobs())} lone GEMVs in a graph: {mc:.4f} ms/step, {chain['alg_GBps']} GB/s")
        del g
    roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "traffic": TRAFFIC_BYTES_PER_STEP if args.layers == LAYERS else None,
                "kernel": "vx::gemv_kernel (one plan run: all 160 projections of a token; event-timed region also "
                          "holds the K-slice finish kernel)",
                "alg_bytes_per_launch": int(st.alg_bytes)}
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline {cpu['value']} Gweights/s")
    plan.close()
    st.free()
    line = {
        "metric": METRIC, "value": round(gw, 1), "unit": "Gweights/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(gw / REF_CPU_GWEIGHTS, 2), "dtype": "int32", "data": "synthetic",
        "config": {"workload": "falcon3-10b-decode-projection-stream (BASELINE.json configs[1])", "layers": args.layers,
                   "hidden": HIDDEN, "ffn": FFN, "kv_rows": KV, "batch": 1, "weights_per_step": st.weights,
                   "gemvs_per_step": len(LAYER_SHAPES) * args.layers, "parallelism": "single-gpu"},
        "hbm_alg_GBps": round(gbps, 1), "hbm_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "device_layout_GBps": round(st.device_bytes / (ms / 1e3) / 1e9, 1),
        "tok_s_projection_bound": round(1e3 / ms, 1),
        "vs_baseline_ref": f"{REF_CPU_GWEIGHTS} Gweights/s, the published Falcon3-10B weight-stream rate of the reference AVX-512 kernel, 4 threads, EPYC 9V45 "
                                   f"(docs/benchmarks.md:77)",
        "chain": chain, "breakdown": breakdown, "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
