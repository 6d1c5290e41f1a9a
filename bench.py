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
MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix peak
LAYERS, HIDDEN, FFN, KV = 40, 3072, 23040, 1024
# (name, rows, cols): the launches of one layer; q|k|v stacked, gate|up interleaved row by row.
LAYER_SHAPES = [("qkv", HIDDEN + 2 * KV, HIDDEN), ("o", HIDDEN, HIDDEN), ("gate_up", 2 * FFN, HIDDEN),
                ("down", HIDDEN, FFN)]
REF_CPU_GWEIGHTS = 221.6  # quintrit_512, 4 threads, EPYC 9V45 (docs/benchmarks.md:77)
# HBM bytes of one full-step gemv_kernel launch, from rocprofv3 FETCH_SIZE and WRITE_SIZE scaled by a plain-copy
# calibration (profiles/gemv_kernel_falcon3_projection_stream.md). Only valid for the default 40-layer workload.
TRAFFIC_BYTES_PER_STEP = 1_902_252 * 1024
SETTLE_S = 0.3  # seconds of back-to-back plan runs before the warm-up steps of the headline timing


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=LAYERS, help=argparse.SUPPRESS)  # smoke runs only
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="leave the decode/prefill measurements out of the line")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave BASELINE.json configs[0], [2] and [4] out of the default line")
    ap.add_argument("--workload", choices=["stream", "gemm", "q2", "decode", "gguf"], default="stream",
                    help="stream: the driver's line (configs[1]); gemm: the batched GEMM of configs[2]; q2: the "
                         "block-scaled GEMV stream of configs[4]; decode: bs=1 greedy decode of configs[3]")
    ap.add_argument("--decode-new", type=int, default=256, help="decode mode: generated tokens per run")
    ap.add_argument("--prefill-tokens", type=int, default=0,
                    help="decode mode: only time the prefill of a prompt of this many tokens")
    ap.add_argument("--model", choices=["bitnet-2b", "falcon3-10b"], default="bitnet-2b",
                    help="decode mode: BASELINE.json configs[3]'s BitNet-2B, or a Falcon3-10B-shaped model (configs[1])")
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


def planar_trits_np(planar, rows: int, cols: int):
    """Trits (int8, rows x cols) of planar velurex bytes (pack.rs:10-16: byte j of block b holds columns
    b*160 + p*32 + j, p = 0..4; B = d0 + 3 d1 + 9 d2 + 28 d3 + 84 d4, t = d - 1), decoded with numpy alone."""
    import numpy as np
    nb = (cols + 159) // 160
    b = np.asarray(planar, np.uint8).reshape(rows, nb, 32).astype(np.int16)
    u = b // 28
    lo = b - 28 * u
    d = np.stack([lo % 3, (lo // 3) % 3, lo // 9, u % 3, u // 3], axis=2)  # rows x nb x 5 x 32
    return (d.reshape(rows, nb * 160)[:, :cols] - 1).astype(np.int8)


def check_outputs_np(st, layer_ids) -> int:
    """Every fp32 output of the given layers of the stream against a numpy brute force of the same planar bytes and
    int8 inputs: acc = sum t x in int64, out = float32(acc) * (float32(0.02) / scale) (the layer epilogue, layer.rs:
    246-253); returns the number of outputs compared, raises on the first mismatching bit."""
    import numpy as np
    n = 0
    for li in layer_ids:
        for t, (name, rows, cols) in enumerate(LAYER_SHAPES):
            k = li * len(LAYER_SHAPES) + t
            planar, q, s = st.kept[k]
            got = st.outs[k].cpu().numpy()
            post = np.float32(0.02) / np.float32(s)
            for r0 in range(0, rows, 4096):
                r1 = min(rows, r0 + 4096)
                tr = planar_trits_np(planar[r0 * ((cols + 159) // 160) * 32:r1 * ((cols + 159) // 160) * 32], r1 - r0, cols)
                acc = tr.astype(np.int64) @ q.astype(np.int64)
                want = acc.astype(np.float32) * post
                if not np.array_equal(want.view(np.uint32), got[r0:r1].view(np.uint32)):
                    bad = int(np.flatnonzero(want.view(np.uint32) != got[r0:r1].view(np.uint32))[0]) + r0
                    raise RuntimeError(f"layer {li} {name} row {bad}: GPU {got[bad]!r} != numpy {want[bad - r0]!r}")
            n += rows
    return n


class Stream:
    """The 40-layer projection stream resident on the GPU, with one staged input vector per projection. The planar
    bytes and int8 inputs of the layers in `keep` stay on the host for the output check."""

    def __init__(self, torch, L, lib, layers: int, keep=()):
        self.torch, self.L, self.lib = torch, L, lib
        self.kept = {}
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0x5EED)
        self.mats = []      # per layer: list of (name, handle, rows, cols)
        self.staged = []    # per launch: (tensor, nbytes)
        self.luts = []      # per launch: the input's compact activation tables (tensor, nbytes)
        self.q = []         # per launch: the int8 input vector the staged bytes were made from
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
                x = torch.randn(cols, device="cuda", generator=gen, dtype=torch.float32)
                q, s = quantize_i8(torch, x)
                if li in keep:
                    self.kept[k] = (planar.cpu().numpy(), q.cpu().numpy(), s)
                del planar
                nbytes = lib.staged_bytes(cols)
                staged = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
                lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(q.data_ptr()), cols, cols,
                                              ctypes.c_void_p(staged.data_ptr()), nbytes, stream))
                lbytes = lib.compact_lut_bytes(cols)
                lut = torch.empty(lbytes, dtype=torch.int8, device="cuda")
                lib.compact_lut_dev(q.data_ptr(), cols, cols, lut.data_ptr(), lbytes, stream)
                self.scales[k] = s
                row.append((name, h, rows, cols))
                self.q.append(q)
                self.staged.append((staged, nbytes))
                self.luts.append((lut, lbytes))
                self.outs.append(torch.empty(rows, dtype=torch.float32, device="cuda"))
                self.weights += rows * cols
                self.alg_bytes += rows * cols / 5.0
                self.device_bytes += lib.layout(rows, cols)["device_bytes"]
                k += 1
            self.mats.append(row)
        torch.cuda.synchronize()

    def jobs(self, which=None, tables=False, raw=False):
        """vx_gemv_job_t list in model order (all launch types, or only LAYER_SHAPES[which]); with `tables` each job
        reads its input's compact activation tables instead of the staged nibbles; with `raw` each job brings its int8
        input and the plan stages it in every run."""
        out = []
        k = 0
        for row in self.mats:
            for t, (_, h, rows, _) in enumerate(row):
                if which is None or which == t:
                    staged, nbytes = (self.luts if tables else self.staged)[k]
                    out.append(self.lib.GemvJob(out_f32=1, matrix=h.value, staged=staged.data_ptr(), staged_len=nbytes,
                                                act_scale_dev=self.scales.data_ptr() + 4 * k,
                                                out=self.outs[k].data_ptr(), out_capacity=rows,
                                                acts=self.q[k].data_ptr() if raw else None))
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

    def stage_all(self) -> None:
        """Every projection's int8 input staged again (vx_stage_acts_dev, one launch per projection)."""
        st = ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)
        k = 0
        for row in self.mats:
            for _, _, _, cols in row:
                staged, nbytes = self.staged[k]
                self.lib.check(self.L.vx_stage_acts_dev(ctypes.c_void_p(self.q[k].data_ptr()), cols, cols,
                                                        ctypes.c_void_p(staged.data_ptr()), nbytes, st))
                k += 1

    def free(self):
        for row in self.mats:
            for _, h, _, _ in row:
                self.lib.check(self.L.vx_matrix_free(h))


LONE_SHAPES = (("q/o", 3072, 3072), ("k/v", 1024, 3072), ("gate/up", 23040, 3072), ("down", 3072, 23040))


def table_decode_ab(torch, st, plan, stream, args) -> dict:
    """The same 160-projection plan through the compact activation tables (vx_lut_plan_create: U/L split of every
    byte and two table lookups, the reference CPU kernel's decode) against the digit-table plan: every output equal
    bit for bit, then both timed back to back."""
    from quintrit_amd import _lib
    lplan = _lib.LutPlan(st.jobs(tables=True))
    plan.run(stream())
    torch.cuda.synchronize()
    want = [o.clone() for o in st.outs]
    for o in st.outs:
        o.fill_(float("nan"))
    lplan.run(stream())
    torch.cuda.synchronize()
    same = all(torch.equal(a.view(torch.int32), b.view(torch.int32)) for a, b in zip(want, st.outs))
    if not same:
        raise SystemExit("the compact-table plan's outputs differ from the digit-table plan's")
    ml, _ = time_fn(torch, lambda: lplan.run(stream()), max(3, args.steps // 2), 2)
    md, _ = time_fn(torch, lambda: plan.run(stream()), max(3, args.steps // 2), 2)
    lbytes = sum(n for _, n in st.luts)
    out = {"ms_per_step": round(ml, 4), "alg_GBps": round(st.alg_bytes / (ml / 1e3) / 1e9, 1),
           "frac": round(st.alg_bytes / (ml / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
           "digit_ms_per_step": round(md, 4), "work_items": lplan.work_items(), "table_bytes": lbytes,
           "outputs": "all 160 equal the digit-table plan's, bit for bit",
           "note": "A/B of the decode: compact tables (2 LDS lookups + 6.5 VALU per weight byte) vs the digit table "
                   "(1 lookup + 3 VALU); same plan, same inputs, tables built before the timed region"}
    log(f"  compact-table plan: {ml:.4f} ms/step ({out['alg_GBps']} GB/s, {out['frac']:.1%} of peak) vs digit-table "
        f"{md:.4f} ms/step")
    lplan.close()
    return out


def lone_latency(torch, L, lib, reps: int = 200):
    """The drop-in path per call at the Falcon3-10B projection shapes: vx_gemv_f32_dev on device buffers (int8
    activations staged by the call, one stream), as a back-to-back stream of `reps` calls (device time per call, HIP
    events) and as single calls each followed by a stream synchronisation (wall-clock median: the latency a lone
    caller sees); and vx_layer_forward, the TernaryGemvLayer::forward stand-in on host buffers (the same call through a
    pinned buffer that the kernels read and write, the caller waiting on the GEMV's completion flag; wall-clock
    median)."""
    import numpy as np
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x10E)
    out = []
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for name, rows, cols in LONE_SHAPES:
        planar = random_planar(torch, rows, cols, gen)
        h = ctypes.c_void_p()
        lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                         ctypes.c_float(0.02), ctypes.byref(h)))
        del planar
        q, sc = quantize_i8(torch, torch.randn(cols, device="cuda", generator=gen))
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        call = lambda: lib.check(L.vx_gemv_f32_dev(h, ctypes.c_void_p(q.data_ptr()), cols, ctypes.c_float(sc),  # noqa: E731
                                                   ctypes.c_void_p(y.data_ptr()), rows, stream))
        ms, _ = time_fn(torch, call, reps, 20)
        lat = []
        for i in range(220):
            t0 = time.perf_counter()
            call()
            torch.cuda.synchronize()
            if i >= 20:
                lat.append(time.perf_counter() - t0)
        qh = q.cpu().numpy()
        yh = np.empty(rows, np.float32)
        fwd = []
        for i in range(220):
            t0 = time.perf_counter()
            lib.check(L.vx_layer_forward(h, qh.ctypes.data_as(ctypes.c_void_p), cols, ctypes.c_float(sc),
                                         yh.ctypes.data_as(ctypes.c_void_p), rows))
            if i >= 20:
                fwd.append(time.perf_counter() - t0)
        if not np.array_equal(yh, y.cpu().numpy()):
            raise RuntimeError(f"{name}: vx_layer_forward and vx_gemv_f32_dev differ")
        out.append({"shape": name, "rows": rows, "cols": cols, "gemv_f32_dev_stream_us": round(ms * 1e3, 2),
                    "gemv_f32_dev_sync_us": round(float(np.median(lat)) * 1e6, 1),
                    "layer_forward_us": round(float(np.median(fwd)) * 1e6, 1)})
        log(f"  lone {name} {rows}x{cols}: {ms * 1e3:.2f} us/call streamed, {np.median(lat) * 1e6:.1f} us with a sync, "
            f"vx_layer_forward {np.median(fwd) * 1e6:.1f} us")
        lib.check(L.vx_matrix_free(h))
    return out


CFG0_ROTATION_BYTES = 1 << 30  # at least 1 GiB of distinct weight copies: beyond the 256 MB last-level cache


def config0_measure(torch, L, lib, cpu: bool) -> dict:
    """one 2560 x 2560 GEMV, trits i.i.d. with P(-1) = P(+1) = 0.35, x 2560 int8 uniform in
    [-127, 127], weight scale 0.02 and activation scale 1, so y = float(acc) * 0.02; int32 acc and fp32 y. Both outputs
    are checked against a numpy brute force of the same planar bytes first. The matrix is 1.31 MB, so a repeated call
    is cache-resident: its figures are latency (a graph of 100 back-to-back calls, HIP events, and one call followed by
    a synchronisation, wall clock) and Gweights/s. For HBM GB/s the same GEMV runs over 1 GiB of distinct copies of
    the matrix (the reference's method: a pass larger than any cache, docs/benchmarks.md:47-49), as one batched plan
    and as a graph of dependent lone calls."""
    import numpy as np
    rows = cols = 2560
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC0)
    planar = random_planar(torch, rows, cols, gen)
    x = torch.randint(-127, 128, (cols,), dtype=torch.int8, device="cuda", generator=gen)
    h = ctypes.c_void_p()
    lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                     ctypes.c_float(0.02), ctypes.byref(h)))
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    acc = torch.empty(rows, dtype=torch.int32, device="cuda")
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731  (the capture stream too)
    stream = cur()
    call_f32 = lambda: lib.check(L.vx_gemv_f32_dev(h, ctypes.c_void_p(x.data_ptr()), cols, ctypes.c_float(1.0),  # noqa: E731
                                                    ctypes.c_void_p(y.data_ptr()), rows, cur()))
    call_i32 = lambda: lib.check(L.vx_gemv_i32_dev(h, ctypes.c_void_p(x.data_ptr()), cols,  # noqa: E731
                                                    ctypes.c_void_p(acc.data_ptr()), rows, cur()))
    call_f32()
    call_i32()
    torch.cuda.synchronize()
    planar_np = planar.cpu().numpy()
    tr = planar_trits_np(planar_np, rows, cols)
    want = tr.astype(np.int64) @ x.cpu().numpy().astype(np.int64)
    if not np.array_equal(acc.cpu().numpy().astype(np.int64), want):
        raise RuntimeError("config 0: int32 accumulators differ from the numpy brute force")
    wy = want.astype(np.float32) * (np.float32(0.02) / np.float32(1.0))
    if not np.array_equal(y.cpu().numpy().view(np.uint32), wy.view(np.uint32)):
        raise RuntimeError("config 0: fp32 outputs differ from float(acc) * 0.02")
    n_in_graph = 100
    g = capture(torch, lambda: [call_f32() for _ in range(n_in_graph)])
    ms, _ = time_fn(torch, g.replay, 20, 3)
    us_call = ms * 1e3 / n_in_graph
    del g
    lat = []
    for i in range(60):
        t0 = time.perf_counter()
        call_f32()
        torch.cuda.synchronize()
        if i >= 10:
            lat.append(time.perf_counter() - t0)
    w = rows * cols
    out = {"shape": [rows, cols], "weights": w, "weight_bytes": w // 5,
           "checked": "int32 acc and fp32 y = float(acc) * 0.02 equal a numpy brute force, bit for bit",
           "call_us": round(us_call, 3), "call_Gweights_s": round(w / (us_call * 1e-6) / 1e9, 1),
           "call_note": "vx_gemv_f32_dev (activation staging + GEMV + epilogue), 100 calls in one HIP graph, device "
                        "time per call; cache-resident",
           "call_sync_us": round(float(np.median(lat)) * 1e6, 1)}
    # rotation: distinct copies of the same planar bytes, 1 GiB of weights in all
    n_copies = -(-CFG0_ROTATION_BYTES // (w // 5))
    mats = [h]
    for _ in range(n_copies - 1):
        hc = ctypes.c_void_p()
        lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                         ctypes.c_float(0.02), ctypes.byref(hc)))
        mats.append(hc)
    del planar
    nbytes = lib.staged_bytes(cols)
    staged = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    lib.check(L.vx_stage_acts_dev(ctypes.c_void_p(x.data_ptr()), cols, cols, ctypes.c_void_p(staged.data_ptr()),
                                  nbytes, stream))
    one = torch.ones(1, dtype=torch.float32, device="cuda")
    outs = torch.empty((n_copies, rows), dtype=torch.float32, device="cuda")
    jobs = [lib.GemvJob(out_f32=1, matrix=m.value, staged=staged.data_ptr(), staged_len=nbytes,
                        act_scale_dev=one.data_ptr(), out=outs[i].data_ptr(), out_capacity=rows)
            for i, m in enumerate(mats)]
    plan = lib.Plan(jobs)
    mp, _ = time_fn(torch, lambda: plan.run(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), 20, 3)
    torch.cuda.synchronize()
    if not torch.equal(outs[-1], y) or not torch.equal(outs[0], y):
        raise RuntimeError("config 0 rotation: a copy's outputs differ from the single call's")

    def chain():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i, m in enumerate(mats):
            lib.check(L.vx_gemv_staged_f32_dev(m, ctypes.c_void_p(staged.data_ptr()), nbytes, ctypes.c_float(1.0),
                                               ctypes.c_void_p(outs[i].data_ptr()), rows, st))
    g = capture(torch, chain)
    mc, _ = time_fn(torch, g.replay, 5, 2)
    del g
    tot_w = w * n_copies
    out["rotation"] = {"copies": n_copies, "weight_bytes": tot_w // 5,
                       "plan_ms": round(mp, 4), "plan_Gweights_s": round(tot_w / (mp / 1e3) / 1e9, 1),
                       "plan_GBps": round(tot_w / 5 / (mp / 1e3) / 1e9, 1),
                       "plan_frac": round(tot_w / 5 / (mp / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                       "chain_ms": round(mc, 4), "chain_us_per_call": round(mc * 1e3 / n_copies, 3),
                       "chain_GBps": round(tot_w / 5 / (mc / 1e3) / 1e9, 1),
                       "note": "plan: all copies in one vx_plan_run (one staged input); chain: one dependent "
                               "vx_gemv_staged_f32_dev per copy in a HIP graph"}
    log(f"config 0: {us_call:.3f} us/call cached ({out['call_Gweights_s']} Gweights/s), {out['call_sync_us']} us "
        f"with a sync; rotation over {n_copies} copies: plan {out['rotation']['plan_GBps']} GB/s, chain "
        f"{out['rotation']['chain_us_per_call']} us/call")
    plan.close()
    for m in mats:
        lib.check(L.vx_matrix_free(m))
    if cpu:
        out["cpu_baseline"] = config0_cpu_baseline(planar_np, rows, cols, x.cpu().numpy(), want)
    return out


def config0_cpu_baseline(planar, rows, cols, acts, want):
    """configs[0] on the host: the AVX-512 transcription of the reference's production GEMV (oracle/cpu_avx512.c,
    avx512.rs:1526-1626) on the 2560 x 2560 tiles, checked against the brute force, then timed (table build + GEMV per
    call, cache-resident as on the reference's machines) at 1, 2, 4, 8, ... threads up to the process's CPUs; the
    best count is the value."""
    import numpy as np
    from oracle import oracle
    if not oracle.cpu_avx512_supported():
        return None
    L = oracle.lib()
    tiles = oracle.tile64(planar, rows, cols)
    out = np.empty(rows, np.float32)
    scratch = np.empty(int(L.vxc_table_bytes(cols)), np.int8)
    ncpu = len(os.sched_getaffinity(0))
    res = {}
    for th in sorted({t for t in (1, 2, 4, 8, 16, 32, 64, ncpu) if t <= ncpu}):
        call = lambda: L.vxc_gemv(tiles.ctypes.data_as(ctypes.c_void_p), acts.ctypes.data_as(ctypes.c_void_p),  # noqa: E731
                                  rows, cols, out.ctypes.data_as(ctypes.c_void_p), th,
                                  scratch.ctypes.data_as(ctypes.c_void_p))
        call()
        if not np.array_equal(out.astype(np.int64), want):
            raise RuntimeError("config 0 CPU baseline differs from the brute force")
        best = 1e9
        t_end = time.perf_counter() + 1.0
        while time.perf_counter() < t_end:
            t0 = time.perf_counter()
            for _ in range(20):
                call()
            best = min(best, (time.perf_counter() - t0) / 20)
        res[th] = best
    top = min(res, key=lambda t: res[t])
    return {"value": round(rows * cols / res[top] / 1e9, 1), "unit": "Gweights/s", "cores": top, "kind": "port",
            "us_per_call": {str(t): round(v * 1e6, 2) for t, v in res.items()},
            "sample": "2560x2560 GEMV (table build + kernel), best of 20-call averages over 1 s per thread count"}


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


def _cpu_model() -> str:
    """/proc/cpuinfo's model name with its family / model / stepping and cache line (a VM may show a short name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k in ("model name", "cpu family", "model", "stepping", "cache size") and k not in info:
                    info[k] = v.strip()
                if not line.strip() and info:
                    break
    except OSError:
        return "unknown"
    return (f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model {info.get('model', '?')}, "
            f"stepping {info.get('stepping', '?')}, cache {info.get('cache size', '?')})")


def _core_order() -> list:
    """The usable logical CPUs, one per physical core first (by package and core id), then their SMT siblings."""
    allowed = sorted(os.sched_getaffinity(0))
    seen, first, rest = set(), [], []
    cpu = phys = None
    topo = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    cpu = int(v)
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    topo[cpu] = (phys, v)
    except OSError:
        return allowed
    for c in allowed:
        key = topo.get(c, (None, c))
        (rest if key in seen else first).append(c)
        seen.add(key)
    return first + rest


def _physical_cores() -> int:
    """Distinct (physical id, core id) pairs in /proc/cpuinfo among the CPUs this process may use."""
    allowed = os.sched_getaffinity(0)
    cores, cpu, phys = set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    cpu = int(v)
                elif k == "physical id":
                    phys = v
                elif k == "core id" and cpu in allowed:
                    cores.add((phys, v))
    except OSError:
        return len(allowed)
    return len(cores) or len(allowed)


def cpu_baseline(budget_s: float, layers: int = 40):
    """The reference's production CPU GEMV (gemv_compact_multi::<3, 4096, T0, 0, true>, avx512.rs:1526-1626 with the
    compact tables of avx512.rs:1216-1247), transcribed with AVX-512 intrinsics (oracle/cpu_avx512.c), timed on this
    host with the reference's method (docs/benchmarks.md:43-59): the Falcon3-10B stream in model order (q, k, v, o,
    gate, up, down) over `layers` distinct layers (40: one whole decode step, 1.9 GB of tiles, far beyond any last-level
    cache), in the engine's call structure: one table build per projection group sharing an input (q/k/v, o, gate/up,
    down) and the group's blocks split over one pool (layer.rs:657-716); threads pinned from C (one per physical core
    first),
    the best of 9 passes per thread count in two rounds, the second in the reverse order, averaged; the read-only memory
    ceiling measured at each thread count in the same session. The transcription is first checked against the
    brute-force product on one 64-row block of every shape. Falls back to the scalar restatement (1 thread) on hosts
    without AVX-512 VBMI. `budget_s` caps the passes of a point once the first is done."""
    import numpy as np
    ncpu, phys = len(os.sched_getaffinity(0)), _physical_cores()
    order = _core_order()
    main_affinity = os.sched_getaffinity(0)
    from oracle import oracle
    L = oracle.lib()
    shapes = [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    if not oracle.cpu_avx512_supported():
        return cpu_baseline_scalar(budget_s, shapes)
    for i, (r, c) in enumerate(shapes):  # exactness of the transcription, every shape
        t = oracle.gen_trits(300 + i, (64, c))
        a = oracle.gen_i8(400 + i, c, -127, 127)
        got = oracle.gemv_avx512(oracle.tile64(oracle.pack_matrix(t), 64, c), a, 64, c, 2)
        if not np.array_equal(got.astype(np.int64), oracle.gemv_bruteforce(t, a)):
            raise RuntimeError(f"AVX-512 transcription differs from the brute-force product at {r}x{c}")
    rng = np.random.default_rng(0xCB)
    # the engine's projection groups, each sharing one input and one table build: q/k/v, o, gate/up, down
    group_of = ((0, 1, 2), (3,), (4, 5), (6,))
    groups, keep = [], []
    for li in range(layers):
        for members in group_of:
            c = shapes[members[0]][1]
            rows = [shapes[m][0] for m in members]
            tiles = [np.empty(r * oracle.tile_row_bytes(c), np.uint8) for r in rows]
            for t in tiles:  # random valid bytes
                L.vxc_fill_valid(t.ctypes.data_as(ctypes.c_void_p), t.size, int(rng.integers(1 << 62)))
            acts = rng.integers(-127, 128, c, dtype=np.int16).astype(np.int8)
            outs = [np.empty(r, np.float32) for r in rows]
            scratch = np.empty(int(L.vxc_table_bytes(c)), np.int8)
            n = len(rows)
            tp = (ctypes.c_void_p * n)(*[t.ctypes.data for t in tiles])
            op = (ctypes.c_void_p * n)(*[o.ctypes.data for o in outs])
            rp = (ctypes.c_size_t * n)(*rows)
            keep.append((tiles, outs))
            groups.append((ctypes.cast(tp, ctypes.c_void_p), ctypes.cast(rp, ctypes.c_void_p), n,
                           acts.ctypes.data_as(ctypes.c_void_p), c, ctypes.cast(op, ctypes.c_void_p),
                           scratch.ctypes.data_as(ctypes.c_void_p), tp, op, rp, acts, scratch))
    weights = layers * sum(r * c for r, c in shapes)
    wbytes = sum(t.size for tiles, _ in keep for t in tiles)
    counts = sorted({t for t in (1, 2, 4, 8, 16, 32, 64, ncpu) if t <= ncpu})
    cpus = (ctypes.c_int * len(order))(*order)

    def one_pass(th):
        t0 = time.perf_counter()
        for tp, rp, n, ap, c, op, sp, *_ in groups:
            L.vxc_gemv_group(tp, rp, n, ap, c, op, th, sp)
        return time.perf_counter() - t0

    buf = np.ones((1 << 30) // 8, np.uint64)
    best = {t: [float("inf"), float("inf")] for t in counts}
    ceiling = {}
    pinned_ok = True
    t_all = time.perf_counter()
    try:
        for rnd, seq in enumerate((counts, counts[::-1])):
            for th in seq:
                pinned_ok &= L.vxc_pin_threads(ctypes.cast(cpus, ctypes.c_void_p), th) == 0
                rb = float("inf")  # the read-only ceiling at this thread count: best of 5 in each round
                for _ in range(5):
                    t0 = time.perf_counter()
                    L.vxc_read_stream(buf.ctypes.data_as(ctypes.c_void_p), buf.size, th)
                    rb = min(rb, time.perf_counter() - t0)
                ceiling[th] = max(ceiling.get(th, 0.0), buf.nbytes / rb / 1e9)
                t0 = time.perf_counter()
                for k in range(9):
                    best[th][rnd] = min(best[th][rnd], one_pass(th))
                    if time.perf_counter() - t0 > budget_s / (2 * len(counts)):
                        break
    finally:
        os.sched_setaffinity(0, main_affinity)  # the pinning moved this (the calling) thread too
    # cache-resident kernel rate of one thread (the reference compares 58-65 weights per cycle for this kernel on
    # cache-resident weights, docs/benchmarks.md:90-92): a 1024 x 3072 projection (630 KB of tiles) from its tables,
    # best of repeated calls, against the core clock measured on the same thread
    pinned_ok &= L.vxc_pin_threads(ctypes.cast(cpus, ctypes.c_void_p), 1) == 0
    try:
        ctile = np.empty(KV * oracle.tile_row_bytes(HIDDEN), np.uint8)
        L.vxc_fill_valid(ctile.ctypes.data_as(ctypes.c_void_p), ctile.size, 17)
        cact = rng.integers(-127, 128, HIDDEN, dtype=np.int16).astype(np.int8)
        ctab = np.empty(int(L.vxc_table_bytes(HIDDEN)), np.int8)
        cout = np.empty(KV, np.float32)
        L.vxc_build_tables(cact.ctypes.data_as(ctypes.c_void_p), HIDDEN, ctab.ctypes.data_as(ctypes.c_void_p))
        cbest = float("inf")
        for _ in range(200):
            t0 = time.perf_counter()
            L.vxc_gemv_tables(ctile.ctypes.data_as(ctypes.c_void_p), ctab.ctypes.data_as(ctypes.c_void_p), KV, HIDDEN,
                              cout.ctypes.data_as(ctypes.c_void_p), 1)
            cbest = min(cbest, time.perf_counter() - t0)
        clock_hz = max(L.vxc_clock_hz() for _ in range(3))
    finally:
        os.sched_setaffinity(0, main_affinity)
    cached_wpc = KV * HIDDEN / cbest / clock_hz
    tab = float("inf")  # the serial part of a pass: the groups' table builds alone (one thread, as the engine's)
    for _ in range(3):
        t0 = time.perf_counter()
        for _tp, _rp, _n, ap, c, _op, sp, *_ in groups:
            L.vxc_build_tables(ap, c, sp)
        tab = min(tab, time.perf_counter() - t0)
    rate = {t: weights / ((best[t][0] + best[t][1]) / 2) / 1e9 for t in counts}  # mean of the two rounds' bests
    top = max(counts, key=lambda t: rate[t])
    wgbps = {t: wbytes / ((best[t][0] + best[t][1]) / 2) / 1e9 for t in counts}
    return {"value": round(rate[top], 1), "unit": "Gweights/s", "cores": top, "kind": "port",
            "sample": f"Falcon3-10B stream in model order over {layers} distinct layers ({weights} weights, "
                      f"{wbytes / 1e6:.0f} MB of 64-row tiles per pass), AVX-512 transcription of the reference's "
                      f"compact_multi_block (NB 3, 4 KiB prefetch) in the engine's projection groups (q/k/v, o, "
                      f"gate/up, down: one table build each, the group's blocks split over the threads); threads "
                      f"{counts} pinned "
                      f"one per core first, best of up to 9 passes per count in two rounds (the second reversed), "
                      f"averaged; {time.perf_counter() - t_all:.1f} s",
            "sweep_gweights_s": {str(t): round(rate[t], 1) for t in counts},
            "weight_GBps": {str(t): round(wgbps[t], 1) for t in counts},
            "read_ceiling_GBps": {str(t): round(ceiling[t], 1) for t in counts},
            "share_of_ceiling": {str(t): round(wgbps[t] / ceiling[t], 3) for t in counts},
            "table_build_ms_per_pass": round(tab * 1e3, 2),
            "table_build_share": {str(t): round(tab / ((best[t][0] + best[t][1]) / 2), 3) for t in counts},
            "threads_pinned": bool(pinned_ok), "cpu_model": _cpu_model(), "logical_cpus": ncpu,
            "physical_cores": phys, "clock_ghz_1t": round(clock_hz / 1e9, 3),
            "cached_1t": {"shape": [KV, HIDDEN], "us": round(cbest * 1e6, 2),
                          "gweights_s": round(KV * HIDDEN / cbest / 1e9, 1),
                          "weights_per_cycle": round(cached_wpc, 1),
                          "reference": "58-65 weights per cycle, cache-resident, EPYC 9V45 (docs/benchmarks.md:90-92)"}}


def cpu_baseline_scalar(budget_s: float, shapes):
    """The CPU oracle's scalar restatement of the reference's table GEMV (oracle/velurex_oracle.c), one thread, over
    the seven projections of one Falcon3-10B layer repeated until the budget is used (hosts without AVX-512 VBMI)."""
    import numpy as np
    from oracle import oracle
    L = oracle.lib()
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
            "sample": f"{reps} pass(es) over the 7 projections of one Falcon3-10B layer, scalar C restatement of the "
                      f"table kernel (no AVX-512 VBMI on this host), 1 thread, {dt:.1f} s"}


def gemm_bench(torch, L, lib, args) -> int:
    """BASELINE.json configs[2] alone: one JSON line with every (shape, M) result and the CPU baseline."""
    results = gemm_measure(torch, L, lib, max(5, args.steps), max(2, args.warmup))
    cpu = None if args.no_cpu_baseline else gemm_cpu_baseline(args.cpu_seconds)
    print(json.dumps({"workload": "batched ternary GEMM, BASELINE.json configs[2]", "dtype": "int8 x ternary -> int32",
                      "data": "synthetic", "note": "device time per vx_gemm_i32_dev call (activation staging + GEMM + "
                      "K-slice finish), HIP events over replays of a graph of 10 calls", "results": results, "cpu_baseline": cpu}), flush=True)
    return 0


def gemm_measure(torch, L, lib, steps: int, warmup: int) -> list:
    """Y = X W^T for W 23040 x 3072 and 3072 x 23040 (velurex), X M x K int8 quantized per
    token from N(0,1), M in {8, 32, 128, 512}; exact int32 on the matrix cores. Every output of one M per shape is
    checked against a float64 brute force of the same planar bytes first (exact: integer operands, |sums| < 2^53).
    ops = 2 M N K; bytes = weights (N K / 5) + X + Y."""
    import numpy as np
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC2)
    results = []
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rows, cols in ((23040, 3072), (3072, 23040)):
        planar = random_planar(torch, rows, cols, gen)
        h = ctypes.c_void_p()
        lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                         ctypes.c_float(0.02), ctypes.byref(h)))
        trits = planar_trits_np(planar.cpu().numpy(), rows, cols).astype(np.float64)
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
                                                       ctypes.c_void_p(ws.data_ptr()), n.value,
                                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
            if m == 32:
                call()
                torch.cuda.synchronize()
                want = q.cpu().numpy().astype(np.float64) @ trits.T
                if not np.array_equal(y.cpu().numpy().astype(np.float64), want):
                    raise RuntimeError(f"gemm {rows}x{cols} m={m}: GPU differs from the float64 brute force")
            # device time per call: 10 calls in one HIP graph (a call is up to three launches, which the host
            # enqueues more slowly than the GPU runs them at small M)
            g = capture(torch, lambda: [call() for _ in range(10)])
            ms, _ = time_fn(torch, g.replay, steps, warmup)
            ms /= 10.0
            del g
            ops = 2.0 * m * rows * cols
            byts = rows * cols / 5.0 + m * cols + 4.0 * m * rows
            r = {"rows": rows, "cols": cols, "m": m, "us": round(ms * 1e3, 2), "TOPS": round(ops / (ms / 1e3) / 1e12, 2),
                 "GBps": round(byts / (ms / 1e3) / 1e9, 1)}
            # the bound: HBM when the weight stream takes longer at 8 TB/s than the operations at the int8 dense peak
            hbm_bound = byts / (HBM_PEAK_GBPS * 1e9) >= ops / (MFMA_I8_PEAK_TOPS * 1e12)
            ach = r["GBps"] if hbm_bound else r["TOPS"]
            peak = HBM_PEAK_GBPS if hbm_bound else MFMA_I8_PEAK_TOPS
            r["roofline"] = {"bound": "hbm" if hbm_bound else "mfma", "achieved": ach, "peak": peak,
                             "unit": "GB/s" if hbm_bound else "TOP/s", "frac": round(ach / peak, 4)}
            log(f"gemm {rows}x{cols} m={m}: {r['us']} us, {r['TOPS']} TOPS, {r['GBps']} GB/s")
            results.append(r)
        lib.check(L.vx_matrix_free(h))
        del trits
    return results


def gemm_cpu_baseline(budget_s: float):
    """The reference has no multi-token kernel: its prefill runs one GEMV per token (quintrit-runtime/src/engine.rs:
    625-631), so its CPU rate for M tokens is M calls of the production AVX-512 GEMV (oracle/cpu_avx512.c, the
    transcription of avx512.rs:1526-1626). Timed for M = 8 tokens on both configs[2] shapes at the thread count that
    is fastest for them (swept 1 .. all CPUs), best of repeated passes within the budget."""
    import numpy as np
    from oracle import oracle
    if not oracle.cpu_avx512_supported():
        return None
    L = oracle.lib()
    rng = np.random.default_rng(0xC2C)
    valid = np.array([b for b in range(256) if oracle.byte_is_valid(b)], np.uint8)
    mats = []
    for r, c in ((23040, 3072), (3072, 23040)):
        tiles = valid[rng.integers(0, valid.size, r * oracle.tile_row_bytes(c), dtype=np.uint16)]
        acts = rng.integers(-127, 128, (8, c), dtype=np.int16).astype(np.int8)
        mats.append((tiles, acts, r, c, np.empty(r, np.float32), np.empty(int(L.vxc_table_bytes(c)), np.int8)))
    ncpu = len(os.sched_getaffinity(0))
    counts = sorted({t for t in (1, 4, 8, 16, 32, 64, ncpu) if t <= ncpu})

    def one_pass(th):
        t0 = time.perf_counter()
        for tiles, acts, r, c, out, scratch in mats:
            for m in range(acts.shape[0]):
                L.vxc_gemv(tiles.ctypes.data_as(ctypes.c_void_p), acts[m].ctypes.data_as(ctypes.c_void_p), r, c,
                           out.ctypes.data_as(ctypes.c_void_p), th, scratch.ctypes.data_as(ctypes.c_void_p))
        return time.perf_counter() - t0

    best = {}
    t_all = time.perf_counter()
    for th in counts:
        best[th] = one_pass(th)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s / (2 * len(counts)):
            best[th] = min(best[th], one_pass(th))
    top = min(counts, key=lambda t: best[t])
    ops = sum(2.0 * acts.shape[0] * r * c for _, acts, r, c, _, _ in mats)
    return {"value": round(ops / best[top] / 1e12, 4), "unit": "TOP/s", "cores": top, "kind": "port",
            "sample": f"M = 8 tokens as 8 AVX-512 GEMV calls (the reference's per-token prefill) on 23040x3072 and "
                      f"3072x23040, threads swept {counts}, best pass at {top}; {time.perf_counter() - t_all:.1f} s",
            "ms_per_pass_at_best": round(best[top] * 1e3, 3)}


Q2_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]


def q2_bench(torch, L, lib, args) -> int:
    """BASELINE.json configs[4] alone: one JSON line with the stream's rate and the CPU baseline."""
    layers = 36 if args.layers == LAYERS else args.layers
    r = q2_measure(torch, L, lib, layers, args.steps, args.warmup)
    r["cpu_baseline"] = None if args.no_cpu_baseline else q2_cpu_baseline(args.cpu_seconds, Q2_SHAPES)
    print(json.dumps(r), flush=True)
    return 0


def q2_measure(torch, L, lib, layers: int, steps: int, warmup: int) -> dict:
    """the projections of one Qwen3-8B-like token (36 layers; q, o 4096 x 4096; k, v
    1024 x 4096; gate, up 12288 x 4096; down 4096 x 12288) as Q2_0 GEMVs: velurex trits plus one fp16 scale per 64
    weights (log-uniform in [0.005, 0.05]) stored beside them, Q8_0 activations (int8 uniform in [-127, 127], one f32
    scale per 32, log-uniform in [0.005, 0.05]). One step = one plan run over all 252 projections."""
    import numpy as np
    shapes = Q2_SHAPES
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
    ms, _ = time_fn(torch, lambda: plan.run(stream()), steps, warmup)
    alg = weights / 5.0 + 2.0 * weights / 64.0
    r = {"workload": "Q2_0 projection stream, BASELINE.json configs[4]", "layers": layers, "weights": weights,
         "ms_per_step": round(ms, 4), "Gweights_s": round(weights / (ms / 1e3) / 1e9, 1),
         "alg_bytes": int(alg), "alg_GBps": round(alg / (ms / 1e3) / 1e9, 1),
         "device_bytes": dev_bytes, "device_GBps": round(dev_bytes / (ms / 1e3) / 1e9, 1),
         "tok_s_projection_bound": round(1e3 / ms, 1), "data": "synthetic", "dtype": "int8 x ternary, fp32 chains"}
    r["roofline"] = {"bound": "hbm", "achieved": r["alg_GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(r["alg_GBps"] / HBM_PEAK_GBPS, 4),
                     "kernel": "vx::q2_kernel (one plan run: all 252 projections of a token)"}
    log(f"q2 stream: {ms:.4f} ms/step, {r['Gweights_s']} Gweights/s, {r['alg_GBps']} GB/s algorithmic")
    plan.close()
    for m in mats:
        m.close()
    return r


def q2_cpu_baseline(budget_s: float, shapes):
    """The reference's Q2_0 x Q8_0 product by its definition (dot_row_scalar, quintrit-core/src/block_scaled.rs:175-202,
    restated in oracle/velurex_oracle.c), rows split over OpenMP threads, over the seven projections of one
    Qwen3-8B-like layer repeated until the budget is used. The reference's own AVX-512 path (block_scaled.rs:495-597) is
    not transcribed, so this is the definition's rate, not the reference's best."""
    import numpy as np
    from oracle import oracle
    rng = np.random.default_rng(0xC4C)
    valid = np.array([b for b in range(256) if oracle.byte_is_valid(b)], np.uint8)
    mats = []
    for r, c in shapes:
        packed = valid[rng.integers(0, valid.size, r * oracle.planar_row_bytes(c), dtype=np.uint16)]
        ws = np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=r * c // 64)).astype(np.float32)
        acts = rng.integers(-127, 128, c, dtype=np.int16).astype(np.int8)
        a_s = np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=c // 32)).astype(np.float32)
        mats.append((packed, ws, acts, a_s, r, c))
    weights, t0, reps = 0, time.perf_counter(), 0
    while True:
        for packed, ws, acts, a_s, r, c in mats:
            oracle.q2_0_gemv(packed, ws, acts, a_s, r, c)
            weights += r * c
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(weights / dt / 1e9, 3), "unit": "Gweights/s", "cores": threads, "kind": "port",
            "sample": f"{reps} pass(es) over the 7 projections of one Qwen3-8B-like layer by the scalar C restatement "
                      f"of dot_row_scalar, {threads} OpenMP threads over rows, {dt:.1f} s"}


def synth_bitnet_planar(np, rng, rows: int, cols: int):
    """Planar velurex bytes (pack.rs:66-131) of i.i.d. trits, P(-1) = P(+1) = 0.35, on the host: each byte of a full
    160-trit block is drawn from the distribution of its five digits (a 65536-entry inverse-CDF table); bytes of the
    last, partial block carry zero trits past `cols`."""
    p = np.array([0.35, 0.30, 0.35])
    digits = np.stack(np.meshgrid(*[np.arange(3)] * 5, indexing="ij"), -1).reshape(-1, 5)  # d0..d4
    prob = np.prod(p[digits], axis=1)
    byte = digits @ np.array([1, 3, 9, 28, 84])
    cdf = np.cumsum(prob)
    table = byte[np.minimum(np.searchsorted(cdf, (np.arange(65536) + 0.5) / 65536.0), len(byte) - 1)].astype(np.uint8)
    nb = (cols + 159) // 160
    out = table[rng.integers(0, 65536, rows * nb * 32, dtype=np.uint16)].reshape(rows, nb, 32)
    rem = cols - (nb - 1) * 160
    if rem < 160:  # trits p*32 + j >= rem of the last block are zero (digit 1)
        v = out[:, nb - 1, :].astype(np.int64)
        dig = np.empty((rows, 5, 32), np.int64)
        u = v // 28
        lo = v - 28 * u
        dig[:, 0], dig[:, 1], dig[:, 2] = lo % 3, (lo // 3) % 3, lo // 9
        dig[:, 3], dig[:, 4] = u % 3, u // 3
        col = np.arange(5)[:, None] * 32 + np.arange(32)[None, :]
        dig[:, col >= rem] = 1
        out[:, nb - 1, :] = (dig * np.array([1, 3, 9, 28, 84])[None, :, None]).sum(1).astype(np.uint8)
    return out.reshape(-1)


def synth_bf16(np, rng, n: int, sigma: float):
    """bf16 bits of N(0, sigma) values (round to nearest even)."""
    out = np.empty(n, np.uint16)
    step = 1 << 24
    for i in range(0, n, step):
        x = (rng.standard_normal(min(step, n - i), dtype=np.float32) * np.float32(sigma)).view(np.uint32)
        out[i:i + x.size] = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    return out


def synth_f16(np, rng, n: int, sigma: float):
    """f16 bits of N(0, sigma) values (round to nearest even)."""
    out = np.empty(n, np.uint16)
    step = 1 << 24
    for i in range(0, n, step):
        x = rng.standard_normal(min(step, n - i), dtype=np.float32) * np.float32(sigma)
        out[i:i + x.size] = x.astype(np.float16).view(np.uint16)
    return out


def decode_cpu_baseline(budget_s: float, prompt, cfg, falcon: bool):
    """The oracle's decode step (oracle/decode_oracle.c: the reference's CPU token loop restated in C, projections
    exact, OpenMP over output rows) on this host's cores, a bounded number of tokens of the same model shape."""
    from oracle import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    m = oracle.Model(oracle.falcon3_10b(cfg.max_ctx, cfg.n_layers) if falcon else oracle.bitnet_2b(cfg.max_ctx), 0xB17)
    t0 = time.perf_counter()
    n = 0
    for pos, tok in enumerate(prompt):
        m.forward(int(tok), pos)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    m.close()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps (positions 0..{n - 1}) of the {'Falcon3-10B' if falcon else 'BitNet-b1.58-2B'}-"
                      f"shaped model by the C restatement of the reference's token loop, {threads} OpenMP threads, "
                      f"{dt:.1f} s"}


def build_decoder_gpu(torch, cfg, seed: int):
    """A random-init decoder of configuration cfg built on the GPU: i.i.d. trits (P(-1) = P(+1) = 0.35) generated in HBM
    and converted there (vx_matrix_create_dev, then vx_decoder_adopt_projection), per-tensor weight scale 1/sqrt(cols),
    norm weights uniform in [0.75, 1.25], embedding (and untied head) N(0, 0.02) in the model's 16-bit type."""
    import numpy as np
    from quintrit_amd import _lib
    from quintrit_amd.decoder import Decoder
    from quintrit_amd.layer import VelurexHipLayer
    L = _lib.lib()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    rng = np.random.default_rng(seed)
    dec = Decoder(cfg)
    trits = 0
    norm_kinds = (0, 1, 2, 3) if cfg.has_sub_norms else (0, 2)
    for layer in range(cfg.n_layers):
        for kind in range(7):
            rows, cols = cfg.projection_shape(kind)
            planar = random_planar(torch, rows, cols, gen)
            h = ctypes.c_void_p()
            _lib.check(L.vx_matrix_create_dev(ctypes.c_void_p(planar.data_ptr()), planar.numel(), rows, cols,
                                              ctypes.c_float(1.0 / float(np.sqrt(np.float32(cols)))), ctypes.byref(h)))
            del planar
            dec.adopt_projection(layer, kind, VelurexHipLayer._from_handle(h))
            trits += rows * cols
        for kind in norm_kinds:
            n = (cfg.hidden, cfg.n_heads * cfg.head_dim, cfg.hidden, cfg.ffn)[kind]
            dec.set_norm(layer, kind, rng.uniform(0.75, 1.25, n).astype(np.float32))
    dec.set_norm(cfg.n_layers, 0, rng.uniform(0.75, 1.25, cfg.hidden).astype(np.float32))
    dt = torch.float16 if cfg.emb_f16 else torch.bfloat16
    for which in ("emb", "head") if cfg.untied else ("emb",):
        t = (torch.randn(cfg.vocab * cfg.hidden, device="cuda", generator=gen) * 0.02).to(dt)
        bits = t.view(torch.int16).cpu().numpy().view(np.uint16)
        del t
        if which == "emb":
            dec.set_embedding(bits)
        else:
            dec.set_head(bits)
    torch.cuda.synchronize()
    return dec, trits


SWEEP_CONTEXTS = (416, 2048, 3900, 7000)  # the reference's published Falcon3-10B context sweep (with its ctx 62)
SWEEP_STEPS = 8


def context_sweep(torch, dec, cfg, runs: int = 2):
    """Decode time per token at the contexts of the reference's Falcon3-10B sweep: a random prompt of ctx tokens
    prefilled, then SWEEP_STEPS + 1 greedy tokens (generate); per token = (generate - prefill alone) / SWEEP_STEPS, the
    steps at positions ctx .. ctx + SWEEP_STEPS - 1. Bytes per step: the trits (0.2 B per weight), the 16-bit head and
    the K and V rows of every cached position (f16)."""
    import numpy as np
    out = []
    kv_row = cfg.n_kv_heads * cfg.head_dim * 2 * 2 * cfg.n_layers  # K and V, f16, every layer
    for ctx in SWEEP_CONTEXTS:
        if ctx + SWEEP_STEPS + 1 > cfg.max_ctx:
            continue
        prompt = np.random.default_rng(ctx).integers(0, cfg.vocab, ctx)
        dec.generate(prompt, SWEEP_STEPS + 1)  # warm-up
        t_pre = t_gen = float("inf")
        for _ in range(runs):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            dec.prefill(prompt, want_logits=False)
            t_pre = min(t_pre, time.perf_counter() - t0)
            t0 = time.perf_counter()
            dec.generate(prompt, SWEEP_STEPS + 1)
            t_gen = min(t_gen, time.perf_counter() - t0)
        ms = (t_gen - t_pre) / SWEEP_STEPS * 1e3
        kv = kv_row * (ctx + SWEEP_STEPS / 2)
        out.append({"ctx": ctx, "ms_per_token": round(ms, 4), "tok_s": round(1e3 / ms, 1),
                    "kv_bytes_per_token": int(kv), "prefill_ms": round(t_pre * 1e3, 2)})
        log(f"context {ctx}: {ms:.4f} ms/token, prefill {t_pre * 1e3:.1f} ms")
    return out


def decode_measure(torch, model: str, n_prompt: int = 64, n_new: int = 256, runs: int = 2, layers: int = 0,
                   sweep: bool = True):
    """Prefill and greedy decode of a random-init model on the GPU (build_decoder_gpu): a 64-token random prompt
    ingested by one prefill (vx_decoder_prefill; the reference feeds it one forward_token per position,
    engine.rs:627-630), then n_new greedy tokens, each one replay of the decode-step graph. Times (wall clock around
    synchronised calls, best of `runs`): the prefill alone, and generation with the prefill, whose difference over the
    n_new - 1 decode steps is the time per token. Rooflines: a decode step streams every trit (0.2 B per weight) and the
    16-bit head; a prefill streams the trits once per pass and does 2 n ops per weight, bound by HBM or the int8
    matrix peak, whichever is slower. The prefill's token also equals the one the step-by-step loop gives (checked)."""
    import numpy as np
    from quintrit_amd.decoder import DecoderConfig
    falcon = model == "falcon3-10b"
    # Falcon3 at the reference GPU decoder's largest context (quintrit-cuda/src/layer.rs:66-67), for the sweep
    cfg = DecoderConfig.falcon3_10b(max_ctx=7936, n_layers=layers or 40) if falcon else DecoderConfig.bitnet_2b()
    log(f"building a random-init {model}-shaped model on the GPU")
    dec, trits = build_decoder_gpu(torch, cfg, 0xB17)
    prompt = np.random.default_rng(0xB17).integers(0, cfg.vocab, n_prompt)
    try:
        _, nxt_pre = dec.prefill(prompt)  # also records the prefill graph
        stepwise = dec.generate(prompt, 1, stepwise=True)
        if stepwise[0] != nxt_pre:
            raise RuntimeError(f"{model}: the prefill's token {nxt_pre} differs from the step-by-step loop's {stepwise[0]}")
        toks = dec.generate(prompt, n_new)  # warm-up, records nothing new
        t_pre = t_gen = float("inf")
        for _ in range(runs):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            dec.prefill(prompt, want_logits=False)
            t_pre = min(t_pre, time.perf_counter() - t0)
            t0 = time.perf_counter()
            again = dec.generate(prompt, n_new)
            t_gen = min(t_gen, time.perf_counter() - t0)
            if again != toks:
                raise RuntimeError(f"{model}: generation is not repeatable")
        ms_tok = (t_gen - t_pre) / max(1, n_new - 1) * 1e3
        sweep_r = context_sweep(torch, dec, cfg) if falcon and sweep else None
    finally:
        dec.close()
    head_bytes = cfg.vocab * cfg.hidden * 2
    alg = trits / 5.0 + head_bytes
    pre_bytes = trits / 5.0 + head_bytes
    pre_ops = 2.0 * n_prompt * trits
    t_hbm, t_mfma = pre_bytes / (HBM_PEAK_GBPS * 1e9), pre_ops / (MFMA_I8_PEAK_TOPS * 1e12)
    pre_s = t_pre
    if t_hbm >= t_mfma:
        pre_roof = {"bound": "hbm", "achieved": round(pre_bytes / pre_s / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(pre_bytes / pre_s / 1e9 / HBM_PEAK_GBPS, 4)}
    else:
        pre_roof = {"bound": "mfma", "achieved": round(pre_ops / pre_s / 1e12, 2), "peak": MFMA_I8_PEAK_TOPS,
                    "unit": "TOP/s", "frac": round(pre_ops / pre_s / 1e12 / MFMA_I8_PEAK_TOPS, 4)}
    r = {"model": model, "layers": cfg.n_layers, "hidden": cfg.hidden, "ffn": cfg.ffn, "vocab": cfg.vocab,
         "trits": trits, "prompt": n_prompt, "new_tokens": n_new,
         "ms_per_token": round(ms_tok, 4), "tok_s": round(1e3 / ms_tok, 1),
         "alg_bytes_per_token": int(alg), "hbm_bound_tok_s": round(HBM_PEAK_GBPS * 1e9 / alg, 1),
         "roofline": {"bound": "hbm", "achieved": round(alg / (ms_tok / 1e3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                      "unit": "GB/s", "frac": round(alg / (ms_tok / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                      "kernel": f"one decode-step graph ({5 * cfg.n_layers + 1} launches); bytes = trits / 5 + head"},
         "prefill_ms": round(t_pre * 1e3, 3), "prefill_tok_s": round(n_prompt / t_pre, 1),
         "prefill_vs_steps": f"{n_prompt} decode steps would take {n_prompt * ms_tok:.2f} ms",
         "prefill_roofline": dict(pre_roof, kernel=f"one prefill pass over {n_prompt} tokens (batched MFMA GEMMs, "
                                  f"per-token norms, attention); bytes = trits / 5 + head, ops = 2 n trits"),
         "generate_ms": round(t_gen * 1e3, 3), "first_tokens": toks[:8]}
    if sweep_r:
        alg_w = trits / 5.0 + head_bytes
        for e in sweep_r:
            b = alg_w + e["kv_bytes_per_token"]
            e["roofline"] = {"bound": "hbm", "achieved": round(b / (e["ms_per_token"] / 1e3) / 1e9, 1),
                             "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                             "frac": round(b / (e["ms_per_token"] / 1e3) / 1e9 / HBM_PEAK_GBPS, 4)}
        r["context_sweep"] = sweep_r
    log(f"{model}: {ms_tok:.4f} ms/token ({1e3 / ms_tok:.1f} tok/s), prefill of {n_prompt} tokens {t_pre * 1e3:.3f} ms")
    return r, cfg, prompt


def decode_bench(torch, args) -> int:
    """--workload decode: prefill and greedy bs=1 decode of a random-init model (decode_measure), one JSON line.
    bitnet-2b    BASELINE.json configs[3]: 30 layers, hidden 2560, 20/5 heads x 128, FFN 6912 ReLU^2, vocab 128256,
                 tied bf16 head
    falcon3-10b  configs[1]'s Falcon3-10B shapes as a whole model: 40 layers, hidden 3072, 12/4 heads x 256, FFN 23040
                 SwiGLU, Normal RoPE, no sub-norms, vocab 131072, f16 embedding and untied f16 head"""
    falcon = args.model == "falcon3-10b"
    if args.prefill_tokens:
        return prefill_bench(torch, args)
    r, cfg, prompt = decode_measure(torch, args.model, n_new=args.decode_new, runs=max(1, args.steps // 10),
                                    layers=args.layers if falcon and args.layers != LAYERS else 0)
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle decode steps)")
        cpu = decode_cpu_baseline(args.cpu_seconds, prompt, cfg, falcon)
        log(f"cpu baseline {cpu['value']} tok/s")
    line = {
        "metric": METRIC, "value": r["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": r["new_tokens"] - 1,
        "warmup": r["new_tokens"], "ms_per_step": r["ms_per_token"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 x ternary, fp32/f16 attention",
        "data": "synthetic (random-init weights, random prompt)",
        "config": {"workload": ("falcon3-10b-shaped greedy decode bs=1 (BASELINE.json configs[1] shapes)" if falcon
                                else "bitnet-b1.58-2b greedy decode bs=1 (BASELINE.json configs[3])"),
                   "layers": cfg.n_layers, "head_dim": cfg.head_dim, "hidden": cfg.hidden, "ffn": cfg.ffn,
                   "vocab": cfg.vocab, "prompt": r["prompt"], "new_tokens": r["new_tokens"],
                   "parallelism": "single-gpu"},
        "decode": r, "roofline": r["roofline"], "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def prefill_bench(torch, args) -> int:
    """--workload decode --prefill-tokens N: the time to ingest an N-token random prompt (vx_decoder_prefill in passes
    of at most 512 tokens, KV cache and last logits as N decode steps would leave them), best of two after a warm-up,
    on the random-init model of --model; one JSON line. A compact command for profiling the prefill kernels."""
    import numpy as np
    from quintrit_amd.decoder import DecoderConfig
    falcon = args.model == "falcon3-10b"
    n = args.prefill_tokens
    max_ctx = max(4096, (n + 255) // 256 * 256)
    if falcon:
        cfg = DecoderConfig.falcon3_10b(max_ctx=max_ctx, n_layers=args.layers if args.layers != LAYERS else 40)
    else:
        cfg = DecoderConfig.bitnet_2b(max_ctx=max_ctx)
    dec = build_decoder_gpu(torch, cfg, 7)[0]
    prompt = np.random.default_rng(n).integers(0, cfg.vocab, n)
    dec.prefill(prompt, want_logits=False)  # warm-up (records the pass graphs)
    best = float("inf")
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompt, want_logits=False)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
    log(f"{args.model}: prefill of {n} tokens {best * 1e3:.1f} ms")
    print(json.dumps({"workload": f"{args.model} prefill of a {n}-token prompt", "layers": cfg.n_layers,
                      "prefill_ms": round(best * 1e3, 2), "tok_s": round(n / best, 1), "data": "synthetic"}),
          flush=True)
    dec.close()
    return 0


FALCON3_LAYER = [("q", 3072, 3072), ("k", 1024, 3072), ("v", 1024, 3072), ("o", 3072, 3072), ("gate", 23040, 3072),
                 ("up", 23040, 3072), ("down", 3072, 23040)]


def gguf_bench(torch, args) -> int:
    """GGUF -> velurex transcoding (loading real model files): the seven ternary tensors of one
    Falcon3-10B layer (237.5 Mweights) in I2_S, TQ1_0 and TQ2_0. Reported per type: the device-side conversion of a
    payload resident in HBM into a GEMV matrix (vx_matrix_create_ggml_dev: payload -> planar -> device layout + row
    digit sums), the whole upload of a GGUF file (open, mmap, PCIe copy of the payload, conversion), and the host
    conversion to planar bytes (vx_ggml_to_planar, one thread per core). The CPU baseline is the oracle's restatement of
    the reference's decoders and packer (decode the trits, pack_matrix), single-threaded as a scalar port."""
    import ctypes as ct
    import tempfile

    import numpy as np
    from oracle import oracle
    from quintrit_amd._lib import check, lib
    from quintrit_amd.gguf import GgufFile, ggml_to_planar
    from quintrit_amd.layer import VelurexHipLayer
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    from gguf_writer import build

    rng = np.random.default_rng(0x6606)
    weights = sum(r * c for _, r, c in FALCON3_LAYER)
    results = {}
    tmp = tempfile.mkdtemp()
    trits = {name: rng.integers(-1, 2, (r, c)).astype(np.int8) for name, r, c in FALCON3_LAYER}
    for ty, tname in ((36, "I2_S"), (34, "TQ1_0"), (35, "TQ2_0")):
        pay = {name: (oracle.i2s_pack(t) if ty == 36 else oracle.tq_pack(ty, t.reshape(-1))) for name, t in trits.items()}
        nbytes = sum(p.size for p in pay.values())
        dev = {name: torch.from_numpy(p).cuda() for name, p in pay.items()}
        torch.cuda.synchronize()

        def device_side():
            ms = []
            for name, r, c in FALCON3_LAYER:
                h = ct.c_void_p()
                check(lib().vx_matrix_create_ggml_dev(ty, ct.c_void_p(dev[name].data_ptr()), dev[name].numel(), r, c,
                                                      ct.c_float(1.0), ct.byref(h)))
                ms.append(VelurexHipLayer._from_handle(h))
            for m in ms:
                m.close()
        device_side()
        reps = max(2, args.steps // 10)
        t0 = time.perf_counter()
        for _ in range(reps):
            device_side()
        torch.cuda.synchronize()
        dt_dev = (time.perf_counter() - t0) / reps
        path = os.path.join(tmp, f"layer_{tname}.gguf")
        with open(path, "wb") as f:
            f.write(build([("general.architecture", 8, "falcon3")],
                          [(f"blk.0.{name}.weight", [c, r], ty,
                            pay[name].tobytes() + (np.float32(0.02).tobytes() if ty == 36 else b""))
                           for name, r, c in FALCON3_LAYER]))
        t0 = time.perf_counter()
        with GgufFile(path) as g:
            ms = [g.upload_matrix(f"blk.0.{name}.weight") for name, _, _ in FALCON3_LAYER]
            torch.cuda.synchronize()
            dt_file = time.perf_counter() - t0
            for m in ms:
                m.close()
        os.remove(path)
        t0 = time.perf_counter()
        for name, r, c in FALCON3_LAYER:
            ggml_to_planar(ty, pay[name], r, c)
        dt_host = time.perf_counter() - t0
        results[tname] = {
            "payload_bytes": nbytes, "device_ms": round(dt_dev * 1e3, 3),
            "device_GBps": round(nbytes / dt_dev / 1e9, 1), "device_Gweights_s": round(weights / dt_dev / 1e9, 1),
            "file_upload_ms": round(dt_file * 1e3, 2), "file_upload_GBps": round(nbytes / dt_file / 1e9, 2),
            "host_ms": round(dt_host * 1e3, 1), "host_GBps": round(nbytes / dt_host / 1e9, 2)}
        log(f"{tname}: {nbytes / 1e6:.1f} MB payload; device {dt_dev * 1e3:.2f} ms ({nbytes / dt_dev / 1e9:.1f} GB/s), "
            f"file upload {dt_file * 1e3:.1f} ms, host {dt_host * 1e3:.1f} ms")
        del dev
    cpu = None
    if not args.no_cpu_baseline:
        # the oracle's decode + pack_matrix on one thread over a bounded sample of the layer (the I2_S q, k, v, o)
        t0, n = time.perf_counter(), 0
        while True:
            for name, r, c in FALCON3_LAYER[:4]:
                p = oracle.i2s_pack(trits[name])
                oracle.pack_matrix(oracle.i2s_unpack(p, r, c))
                n += r * c
            if time.perf_counter() - t0 > min(args.cpu_seconds, 8.0):
                break
        dt = time.perf_counter() - t0
        cpu = {"value": round(n / 4 / dt / 1e9, 3), "unit": "GB/s of I2_S payload", "cores": 1, "kind": "port",
               "sample": f"{n / 1e6:.0f} Mweights of the layer's q/k/v/o in I2_S through the oracle's decoder and "
                         f"pack_matrix, one thread, {dt:.1f} s (timing includes the oracle's I2_S re-encode)"}
    head = results["I2_S"]
    line = {
        "metric": "GGUF ternary transcoding to the velurex device layout (Falcon3-10B layer shapes)",
        "value": head["device_GBps"], "unit": "GB/s of I2_S payload", "n_gpus": 1, "steps": max(2, args.steps // 10),
        "warmup": 1, "ms_per_step": head["device_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic (random trits)",
        "config": {"workload": "gguf transcoding: one Falcon3-10B layer (7 tensors, 237.5 Mweights)", "weights": weights},
        "results": results, "cpu_baseline": cpu,
        "roofline": {"bound": "hbm", "achieved": round((weights / 4 + weights / 5) / (head["device_ms"] / 1e3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round((weights / 4 + weights / 5) / (head["device_ms"] / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "kernel": "device-side matrix creation (conversion, check, layout, digit sums and allocations); "
                               "bytes = I2_S payload read + planar written"}}
    print(json.dumps(line), flush=True)
    return 0


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (how the path would shard over "
                                   "several GPUs is a design only, not built)"}))
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
    if args.workload == "decode":
        return decode_bench(torch, args)
    if args.workload == "gguf":
        return gguf_bench(torch, args)
    log(f"building the {args.layers}-layer weight stream on the GPU")
    check_layers = sorted({0, args.layers - 1})
    st = Stream(torch, L, _lib, args.layers, keep=check_layers)
    log(f"{st.weights} weights, {st.alg_bytes / 1e9:.4f} GB algorithmic, {st.device_bytes / 1e9:.4f} GB device layout")
    plan = _lib.Plan(st.jobs())
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    step = lambda: plan.run(stream())  # noqa: E731
    # The plan's outputs of the first and last layer against numpy before anything is timed.
    step()
    torch.cuda.synchronize()
    n_checked = check_outputs_np(st, check_layers)
    log(f"plan outputs of layers {check_layers} equal the numpy brute force ({n_checked} rows)")

    # The other measurements run first: they also bring the GPU to its steady clocks before the headline timing.
    breakdown = {}
    chain = None
    table_decode = None
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
        chain["lone_calls"] = lone_latency(torch, L, _lib)
        table_decode = table_decode_ab(torch, st, plan, stream, args)

    for o in st.outs:
        o.fill_(float("nan"))
    # Settle: the plan runs back to back for SETTLE_S before the warm-up steps, so the timed steps see the GPU's steady
    # clocks (after idle host work, a few warm-up steps alone leave the first timed steps up to 10 % slower).
    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(25):
            step()
        n_settle += 25
        torch.cuda.synchronize()
    log(f"plan: {len(st.jobs())} GEMVs, {plan.work_items()} work items; settled ({n_settle} runs), timing {args.steps} "
        f"steps after {args.warmup}")
    ms, wall = time_fn(torch, step, args.steps, args.warmup)
    gw = st.weights / (ms / 1e3) / 1e9
    gbps = st.alg_bytes / (ms / 1e3) / 1e9
    log(f"{ms:.4f} ms/step, {gw:.1f} Gweights/s, {gbps:.1f} GB/s algorithmic ({gbps / HBM_PEAK_GBPS:.1%} of peak), "
        f"wall {wall / args.steps * 1e3:.4f} ms/step")
    # ... and the outputs of the last timed step, again against numpy (a mismatch fails the run)
    n_checked = check_outputs_np(st, check_layers)
    log(f"after timing: layers {check_layers} still equal the numpy brute force")
    # the same step with every projection's activation staging inside the timed region: a plan whose jobs bring their
    # raw int8 inputs (one staging launch for all 160, then the GEMVs); and, for comparison, 160 separate staging
    # launches before the plan run in one HIP graph
    rplan = _lib.Plan(st.jobs(raw=True))
    for o in st.outs:
        o.fill_(float("nan"))
    msr, _ = time_fn(torch, lambda: rplan.run(stream()), args.steps, args.warmup)
    n_checked += check_outputs_np(st, check_layers[-1:])
    rplan.close()
    g = capture(torch, lambda: (st.stage_all(), step()))
    msg, _ = time_fn(torch, g.replay, max(3, args.steps // 2), 2)
    del g
    with_staging = {"ms_per_step": round(msr, 5), "Gweights_s": round(st.weights / (msr / 1e3) / 1e9, 1),
                    "frac": round(st.alg_bytes / (msr / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                    "note": "each job brings its raw int8 input: every run stages all 160 in one launch, then the GEMVs "
                            "(vx_gemv_job_t.acts); outputs checked against numpy after the timing",
                    "separate_launches_ms_per_step": round(msg, 5)}
    log(f"with the staging in the step: {msr:.4f} ms/step ({with_staging['frac']:.1%} of peak); as 160 separate "
        f"staging launches: {msg:.4f} ms/step")
    roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "traffic": TRAFFIC_BYTES_PER_STEP if args.layers == LAYERS else None,
                "traffic_source": "a constant: rocprofv3 FETCH_SIZE + WRITE_SIZE of this launch, scaled by a plain-copy "
                                  "calibration (profiles/gemv_kernel_falcon3_projection_stream.md), not measured in "
                                  "this run",
                "kernel": "vx::gemv_kernel (one plan run: all 160 projections of a token; event-timed region also "
                          "holds the K-slice finish kernel)",
                "alg_bytes_per_launch": int(st.alg_bytes)}
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline {cpu['value']} Gweights/s")
    n_weights, n_gemvs = st.weights, len(st.jobs())
    dev_gbps = st.device_bytes / (ms / 1e3) / 1e9
    plan.close()
    st.free()
    del st, plan
    torch.cuda.empty_cache()
    config0 = gemm = q2 = None
    if not args.no_configs:
        # BASELINE.json configs[0], [2] and [4] in the same line (each also has a --workload mode of its own)
        config0 = config0_measure(torch, L, _lib, cpu=not args.no_cpu_baseline)
        torch.cuda.empty_cache()
        gemm = [{k: r[k] for k in ("rows", "cols", "m", "us", "TOPS", "GBps")} | {"frac": r["roofline"]["frac"],
                                                                                "bound": r["roofline"]["bound"]}
                for r in gemm_measure(torch, L, _lib, 20, 5)]
        torch.cuda.empty_cache()
        r = q2_measure(torch, L, _lib, 36, 50, 10)
        q2 = {k: r[k] for k in ("layers", "ms_per_step", "Gweights_s", "alg_GBps", "tok_s_projection_bound")}
        q2["frac"] = r["roofline"]["frac"]
        torch.cuda.empty_cache()
    decode = None
    if not args.no_decode:
        # tok/s at bs = 1: both decode models of BASELINE.json (configs[3] BitNet-2B, configs[1]'s Falcon3-10B shapes)
        decode = {}
        for model in ("bitnet-2b", "falcon3-10b"):
            decode[model.replace("-", "_")] = decode_measure(torch, model)[0]
            torch.cuda.empty_cache()
    line = {
        "metric": METRIC, "value": round(gw, 1), "unit": "Gweights/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(gw / REF_CPU_GWEIGHTS, 2), "dtype": "int32", "data": "synthetic",
        "config": {"workload": "falcon3-10b-decode-projection-stream (BASELINE.json configs[1])", "layers": args.layers,
                   "hidden": HIDDEN, "ffn": FFN, "kv_rows": KV, "batch": 1, "weights_per_step": n_weights,
                   "gemvs_per_step": n_gemvs, "parallelism": "single-gpu",
                   "inputs": "resident in HBM; each projection's int8 input quantized and staged (vx_stage_acts_dev) "
                             "before the timed region, the timed step is the GEMVs with their fp32 epilogue"},
        "hbm_alg_GBps": round(gbps, 1), "hbm_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "device_layout_GBps": round(dev_gbps, 1),
        "tok_s_projection_bound": round(1e3 / ms, 1),
        "checked": {"layers": check_layers, "rows": n_checked, "against": "numpy int64 brute force of the planar bytes "
                    "and the fp32 epilogue, bit for bit, before and after the timed steps"},
        "vs_baseline_ref": f"{REF_CPU_GWEIGHTS} Gweights/s, the published Falcon3-10B weight-stream rate of the reference AVX-512 kernel, 4 threads, EPYC 9V45 "
                                   f"(docs/benchmarks.md:77)",
        "settle": {"seconds": SETTLE_S, "plan_runs": n_settle},
        "with_staging": with_staging,
        "chain": chain, "breakdown": breakdown, "table_decode": table_decode, "roofline": roofline, "cpu_baseline": cpu,
        "config0": config0, "gemm_config2": gemm, "q2_config4": q2, "decode": decode,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
