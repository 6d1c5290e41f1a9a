"""Pins the CPU oracle (oracle/velurex_oracle.c) before anything is checked against it.

Every check here is independent of the formula the oracle implements: round trips, brute force computed with numpy,
closed forms, numpy's own float16 / rounding routines, and the test patterns of the reference's own test suites
(quintrit-core/tests/pack_tests.rs, kernel_tests.rs; quintrit-cuda/tests/gemv.rs:46-64,84-88).
"""
import itertools

import numpy as np
import pytest


RADIX = (1, 3, 9, 28, 84)


# ---- encoding --------------------------------------------------------------------------------------------------------

def test_all_243_states_round_trip(oracle):
    # pack_tests.rs:7-40: every combination of five trits survives pack -> unpack; the bytes are distinct and <= 250.
    seen = set()
    for t in itertools.product((-1, 0, 1), repeat=5):
        b = oracle.pack_5trits(t)
        assert 0 <= b <= 250
        assert tuple(oracle.byte_to_trits(b)) == t
        seen.add(b)
    assert len(seen) == 243
    assert max(seen) == 250 and min(seen) == 0


def test_invalid_bytes_decode_to_zero(oracle):
    # pack_tests.rs:42-53: bytes 251..255 decode to zeros; so do the gap bytes 27, 55, 83, ... (never produced).
    valid = {oracle.pack_5trits(t) for t in itertools.product((-1, 0, 1), repeat=5)}
    for b in range(256):
        assert oracle.byte_is_valid(b) == (b in valid)
        if b not in valid:
            assert not oracle.byte_to_trits(b).any()
    for b in (27, 55, 83, 251, 252, 253, 254, 255):
        assert b not in valid


def test_decode_is_floor_div_28(oracle):
    # docs/velurex-encoding.md section 2: U = floor(B / 28), L = B - 28 U; the table decode must agree on all 243.
    for t in itertools.product((-1, 0, 1), repeat=5):
        b = oracle.pack_5trits(t)
        u, l = oracle.decode_u_l(b)
        assert (u, l) == (b // 28, b % 28)
        d = [x + 1 for x in t]
        assert u == d[3] + 3 * d[4] and l == d[0] + 3 * d[1] + 9 * d[2]


@pytest.mark.parametrize("cols", [1, 31, 32, 159, 160, 161, 320, 3072, 4096])
def test_pack_unpack_round_trip(oracle, cols):
    rng = np.random.default_rng(cols)
    rows = 5
    trits = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    packed = oracle.pack_matrix(trits)
    assert packed.shape == (rows, -(-cols // 160) * 32)
    assert np.array_equal(oracle.unpack_matrix(packed, rows, cols), trits)
    # Planar layout stated in the module doc (pack.rs:10-16): byte j of block b holds columns b*160 + p*32 + j.
    for r in range(rows):
        for c in rng.integers(0, cols, size=8):
            b, rem = divmod(int(c), 160)
            p, j = divmod(rem, 32)
            assert oracle.byte_to_trits(packed[r, b * 32 + j])[p] == trits[r, c]


def test_tile_row_bytes_matches_published_sizes(oracle):
    # Bytes per row at the model widths, planar / tiled, as pack.rs:222-225 sizes them (whole 160-column blocks of 32
    # bytes, then the packed tail of ceil(rest / 5) bytes rounded up to even).
    table = {2560: (512, 512), 3072: (640, 616), 4096: (832, 820), 6912: (1408, 1384), 12288: (2464, 2458),
             23040: (4608, 4608)}
    for cols, (planar, tiled) in table.items():
        assert oracle.planar_row_bytes(cols) == planar
        assert oracle.tile_row_bytes(cols) == tiled


@pytest.mark.parametrize("cols", [1, 2, 5, 6, 159, 161, 165, 3072, 3079])
def test_tile_transform_lossless(oracle, cols):
    # pack_tests.rs:101-130: tile row -> planar row is the identity for every tail length.
    rng = np.random.default_rng(1000 + cols)
    trits = rng.integers(-1, 2, size=(1, cols), dtype=np.int8)
    planar = oracle.pack_matrix(trits)[0]
    tile = oracle.tile_row(planar, cols)
    assert tile.size == oracle.tile_row_bytes(cols)
    assert np.array_equal(oracle.untile_row(tile, cols), planar)
    # Each tile byte holds the trits of the activations column_activation_index names.
    for c in range(tile.size):
        t = oracle.byte_to_trits(tile[c])
        for p in range(5):
            idx = oracle.column_activation_index(cols, c, p)
            assert t[p] == (trits[0, idx] if idx < cols else 0)


@pytest.mark.parametrize("cols", [160, 161, 3072, 23040])
def test_column_activation_index_is_a_bijection(oracle, cols):
    idx = [oracle.column_activation_index(cols, c, p) for c in range(oracle.tile_row_bytes(cols)) for p in range(5)]
    inside = sorted(i for i in idx if i < cols)
    assert inside == list(range(cols))


# ---- activation split and tables -------------------------------------------------------------------------------------

def test_split_hi_lo_all_int8(oracle):
    # kernel_tests.rs:264-273: x = 16 hi + lo with lo in [-8, 7] and hi in [-8, 8] for all 256 values.
    x = np.arange(-128, 128, dtype=np.int8)
    hi, lo = oracle.split_hi_lo(x)
    assert np.array_equal(16 * hi.astype(np.int32) + lo, x.astype(np.int32))
    assert lo.min() == -8 and lo.max() == 7 and hi.min() == -8 and hi.max() == 8


def test_compact_table_entries_are_small(oracle):
    acts = np.array([127, -128] * 80, np.int8)
    lut = oracle.build_compact_wide_lut(acts, 160)
    assert np.abs(lut.astype(np.int32)).max() <= 24  # |entry| <= 3 * 8 (avx512.rs:1210-1213)


# ---- GEMV: the reference's own ground truth is brute force --------------------------------------------------------------

def _weights(kind, rows, cols, rng):
    return {"random": lambda: rng.integers(-1, 2, size=(rows, cols), dtype=np.int8),
            "plus": lambda: np.ones((rows, cols), np.int8),
            "minus": lambda: -np.ones((rows, cols), np.int8),
            "zero": lambda: np.zeros((rows, cols), np.int8)}[kind]()


def _acts(kind, cols, rng):
    return {"random": lambda: rng.integers(-128, 128, size=cols, dtype=np.int8),
            "max": lambda: np.full(cols, 127, np.int8),
            "min": lambda: np.full(cols, -128, np.int8),
            "alternating": lambda: np.where(np.arange(cols) % 2 == 0, 127, -128).astype(np.int8)}[kind]()


def test_bruteforce_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    t = rng.integers(-1, 2, size=(33, 777), dtype=np.int8)
    a = rng.integers(-128, 128, size=777, dtype=np.int8)
    assert np.array_equal(oracle.gemv_bruteforce(t, a), t.astype(np.int64) @ a.astype(np.int64))


@pytest.mark.parametrize("cols", [1, 160, 161, 320, 2560, 3072, 4096])
def test_lut_gemv_equals_bruteforce_pattern_grid(oracle, cols):
    # quintrit-cuda/tests/gemv.rs:77-104 grid: weights {random, +1, -1, 0} x activations {random, 127, -128, alt}.
    rng = np.random.default_rng(cols)
    rows = 8
    for wk in ("random", "plus", "minus", "zero"):
        t = _weights(wk, rows, cols, rng)
        packed = oracle.pack_matrix(t)
        for ak in ("random", "max", "min", "alternating"):
            a = _acts(ak, cols, rng)
            want = t.astype(np.int64) @ a.astype(np.int64)
            got = oracle.gemv_lut_planar(packed, rows, cols, a)
            assert np.array_equal(got.astype(np.int64), want), (wk, ak)


def test_lut_gemv_wide_shape(oracle):
    rng = np.random.default_rng(23040)
    t = rng.integers(-1, 2, size=(4, 23040), dtype=np.int8)
    a = rng.integers(-128, 128, size=23040, dtype=np.int8)
    got = oracle.gemv_lut_planar(oracle.pack_matrix(t), 4, 23040, a)
    assert np.array_equal(got.astype(np.int64), t.astype(np.int64) @ a.astype(np.int64))


def test_epilogue_special_cases(oracle):
    acc = np.array([0, 1, -1, 12345, -(1 << 23), (1 << 24) - 1], np.int32)
    assert np.array_equal(oracle.epilogue_f32(acc, 0.5, 0.5), acc.astype(np.float32))      # ws / as = 1
    assert np.array_equal(oracle.epilogue_f32(acc, 2.0, 0.5), 4 * acc.astype(np.float32))  # power of two
    assert not oracle.epilogue_f32(acc, 0.3, 0.0).any() and not oracle.epilogue_f32(acc, 0.3, -1.0).any()
    # Generic scales: one rounding of the quotient and one of the product -> within 2 ulp of the exact value.
    ws, as_ = 0.02, 0.7
    got = oracle.epilogue_f32(acc, ws, as_).astype(np.float64)
    exact = acc.astype(np.float64) * ws / as_
    assert np.all(np.abs(got - exact) <= 2.5 * np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) + 1e-30)


# ---- quantizers ---------------------------------------------------------------------------------------------------

def test_quantize_i8_properties(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(3072).astype(np.float32)
    q, s = oracle.quantize_i8(x)
    assert s == pytest.approx(127.0 / np.abs(x).max(), rel=1e-7)
    assert q[np.argmax(np.abs(x))] in (127, -127)
    assert np.abs(q.astype(np.float64) - x.astype(np.float64) * s).max() <= 0.5 + 1e-4
    q0, s0 = oracle.quantize_i8(np.zeros(16, np.float32))
    assert s0 == 0.0 and not q0.any()


def test_quantize_i8_rounds_half_away_from_zero(oracle):
    # f32::round (ops.rs:261) rounds halves away from zero; numpy's rint would give 2 and -2 here.
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5], np.float32)
    q, s = oracle.quantize_i8(x)
    assert s == 1.0
    assert list(q) == [127, 3, -3, 1, -1, 2]


def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(9)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-5).astype(np.float32),
        (rng.standard_normal(2000) * 3e4).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 6e-8, 3e-8, 2.98e-8, 5.96e-8, 6.1e-5, np.inf, -np.inf],
                 np.float32),
        # exact halfway points between halves (ties to even)
        (np.arange(1024, 1100, dtype=np.float32) + 0.5).astype(np.float32),
    ])
    for v in vals:
        want = int(np.array(v, np.float32).astype(np.float16).view(np.uint16))
        assert oracle.f32_to_f16_bits(float(v)) == want, v
    for h in list(range(0, 0x7c01, 97)) + [0x0001, 0x03ff, 0x0400, 0x7bff, 0x7c00, 0x8001, 0xfbff]:
        want = float(np.array(h, np.uint16).view(np.float16).astype(np.float32))
        assert oracle.f16_bits_to_f32(h) == want


def test_quantize_q8_0_matches_numpy_definition(oracle):
    # ops.rs:877-910: d = fp16(amax / 127), codes = round_half_even(x * (127 / amax)); numpy rint is half-even.
    rng = np.random.default_rng(11)
    x = rng.standard_normal(32 * 40).astype(np.float32)
    x[32:64] = 0.0
    qs, d = oracle.quantize_q8_0(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    with np.errstate(divide="ignore"):
        idv = np.where(amax != 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    want = np.clip(np.rint(xb * idv[:, None]), -128, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(qs, want)


def test_rms_norm_close_to_float64(oracle):
    rng = np.random.default_rng(13)
    x = rng.standard_normal(3072).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(3072)).astype(np.float32)
    got = oracle.rms_norm(x, w, 1e-6)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(got, ref, rtol=3e-7 * 4, atol=0)
    ones = oracle.rms_norm(np.ones(8, np.float32), np.ones(8, np.float32), 0.0)
    assert np.array_equal(ones, np.ones(8, np.float32))


# ---- Q2_0 -----------------------------------------------------------------------------------------------------------

def test_q2_0_lane_sums_are_exact(oracle):
    rng = np.random.default_rng(17)
    rows, cols = 3, 4096
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    sums = oracle.q2_0_lane_sums(oracle.pack_matrix(t), a, rows, cols)
    want = (t.astype(np.int32) * a.astype(np.int32)).reshape(rows, cols // 32, 8, 4).sum(axis=3)
    assert np.array_equal(sums, want)


def test_q2_0_unit_scales_give_the_integer_dot(oracle):
    # With every scale 1 the chains hold exact integers (|sum| < 2^24), so the result is the exact dot product.
    rng = np.random.default_rng(19)
    rows, cols = 4, 12288
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-128, 128, size=cols, dtype=np.int8)
    got = oracle.q2_0_gemv(oracle.pack_matrix(t), np.ones(rows * cols // 64, np.float32), a,
                           np.ones(cols // 32, np.float32), rows, cols)
    assert np.array_equal(got.astype(np.int64), t.astype(np.int64) @ a.astype(np.int64))


def test_q2_0_close_to_float64(oracle):
    rng = np.random.default_rng(21)
    rows, cols = 6, 4096
    t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    a = rng.integers(-127, 128, size=cols, dtype=np.int8)
    ws = np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=rows * cols // 64)).astype(np.float32)
    as_ = np.exp(rng.uniform(np.log(0.005), np.log(0.05), size=cols // 32)).astype(np.float32)
    got = oracle.q2_0_gemv(oracle.pack_matrix(t), ws, a, as_, rows, cols)
    prod = (t.astype(np.float64) * a.astype(np.float64)).reshape(rows, cols // 32, 32).sum(axis=2)
    d = ws.reshape(rows, cols // 64).astype(np.float64).repeat(2, axis=1) * as_.astype(np.float64)[None, :]
    ref = (prod * d).sum(axis=1)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


# Hand-computed rows for the floating-point order of Q2_0 (block_scaled.rs:1-19,140-145,175-202). cols = 256: eight
# activation blocks s (weight block s / 2, chain (s / 2) & 1), every activation 1, so a lane sum is the sum of four
# trits. f32 has 24 significant bits: 2^24 + 1 is a tie that rounds to 2^24, while 2^24 + 2 is exact.
Q2_ROWS, Q2_COLS = 5, 256


def q2_order_case():
    t = np.zeros((Q2_ROWS, Q2_COLS), np.int8)
    ws = np.ones((Q2_ROWS, Q2_COLS // 64), np.float32)
    as_ = np.ones(Q2_COLS // 32, np.float32)
    # row 0, the two chains: s=0 lane 0 = 2^24 (chain 0); s=2 and s=3 lane 0 = 1 each (chain 1, which holds 2).
    # l0 = 2^24 + 2. One chain: 2^24 + 1 + 1 = 2^24; chains by s & 1: (2^24 + 1) + 1 = 2^24.
    ws[0, 0] = 2.0 ** 24
    t[0, [0, 64, 96]] = 1
    # row 1, hsum8's pairing: l0 = 2^24 (s=0, 4 trits x 2^22), l2 = 1 and l6 = 1 (s=2 lanes 2 and 6).
    # ((l0+l4) + (l2+l6)) + ... = 2^24 + 2. In lane order, or as ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)): 2^24.
    ws[1, 0] = 2.0 ** 22
    t[1, [0, 1, 2, 3, 64 + 8, 64 + 24]] = 1
    # row 2, chains added lane by lane before hsum8: chain 0 lane 0 = 2^24, chain 1 lanes 0 and 4 = 1 each.
    # l0 = 2^24 + 1 = 2^24, l4 = 1, (l0 + l4) = 2^24. hsum8 of each chain, then added: 2^24 + 2.
    ws[2, 0] = 2.0 ** 22
    t[2, [0, 1, 2, 3, 64, 64 + 16]] = 1
    # row 3, the fused multiply-add: s=0 lane 0 = -3 (d = 1); s=1 lane 0 = 3 with d = 1 + 2^-23 (as[1]).
    # fma(1 + 2^-23, 3, -3) = 3 * 2^-23. A rounded product first: f32(3 + 3 * 2^-23) = 3 + 2^-21, so 2^-21.
    as_[1] = np.float32(1 + 2.0 ** -23)
    t[3, [0, 1, 2]] = -1
    t[3, [32, 33, 34]] = 1
    # row 4, d = f32(ws * as) before the lane sum: ws = as = 1 + 2^-12 at s=4, lane 0 = 3.
    # d = f32(1 + 2^-11 + 2^-24) = 1 + 2^-11 (tie to even), 3 d = 3 + 3 * 2^-11 exactly.
    # ws * (as * 3) = f32(3 + 3 * 2^-11 + 3 * 2^-24) = 3 + 3 * 2^-11 + 2^-22.
    ws[4, 2] = np.float32(1 + 2.0 ** -12)
    as_[4] = np.float32(1 + 2.0 ** -12)
    t[4, [128, 129, 130]] = 1
    a = np.ones(Q2_COLS, np.int8)
    want = np.array([2.0 ** 24 + 2, 2.0 ** 24 + 2, 2.0 ** 24, 3 * 2.0 ** -23, 3 + 3 * 2.0 ** -11], np.float32)
    return t, ws, a, as_, want


def q2_definition(t, ws, a, as_, *, chains=2, chain_of_s=None, pairing="ggml", fused=True, scale_first=True,
                  hsum_per_chain=False):
    """The documented order with switches for the negative controls. Products and sums are formed in float64 and
    rounded once to f32, which is exact for these inputs' magnitudes (so fused = one rounding)."""
    f32 = np.float32
    rows, cols = t.shape
    out = np.empty(rows, np.float32)
    for r in range(rows):
        acc = np.zeros((2, 8), np.float32)
        for s in range(cols // 32):
            c = ((s // 2) & 1 if chain_of_s is None else chain_of_s(s)) if chains == 2 else 0
            lanes = (t[r, s * 32:(s + 1) * 32].astype(np.int64) * a[s * 32:(s + 1) * 32]).reshape(8, 4).sum(axis=1)
            for j in range(8):
                p = float(lanes[j])
                if scale_first:
                    d = f32(float(ws[r, s // 2]) * float(as_[s]))
                    prod = float(d) * p
                else:
                    prod = float(ws[r, s // 2]) * float(f32(float(as_[s]) * p))
                if not fused:
                    prod = float(f32(prod))
                acc[c, j] = f32(prod + float(acc[c, j]))

        def hsum(l):
            if pairing == "ggml":
                return f32(f32(f32(l[4] + l[0]) + f32(l[6] + l[2])) + f32(f32(l[5] + l[1]) + f32(l[7] + l[3])))
            if pairing == "sequential":
                s_ = f32(0)
                for x in l:
                    s_ = f32(s_ + x)
                return s_
            return f32(f32(f32(l[0] + l[1]) + f32(l[2] + l[3])) + f32(f32(l[4] + l[5]) + f32(l[6] + l[7])))
        if hsum_per_chain:
            out[r] = f32(hsum(acc[0]) + hsum(acc[1]))
        else:
            out[r] = hsum((acc[0] + acc[1]).astype(np.float32))
    return out


def test_q2_0_order_hand_computed(oracle):
    """The oracle's Q2_0 rows equal the hand-computed values above bit for bit; so does the documented definition."""
    t, ws, a, as_, want = q2_order_case()
    got = oracle.q2_0_gemv(oracle.pack_matrix(t), ws.reshape(-1), a, as_, Q2_ROWS, Q2_COLS)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(q2_definition(t, ws, a, as_).view(np.uint32), want.view(np.uint32))


def test_q2_0_order_negative_controls():
    """Each plausible mistake changes the row built to show it: one accumulator, chains chosen by s & 1, lanes summed in
    order or in adjacent pairs, an unfused multiply-add, the scale applied after the lane sum, hsum8 of each chain."""
    t, ws, a, as_, want = q2_order_case()
    mutants = [
        (dict(chains=1), 0), (dict(chain_of_s=lambda s: s & 1), 0), (dict(pairing="sequential"), 1),
        (dict(pairing="adjacent"), 1), (dict(hsum_per_chain=True), 2), (dict(fused=False), 3),
        (dict(scale_first=False), 4),
    ]
    for kw, row in mutants:
        bad = q2_definition(t, ws, a, as_, **kw)
        assert bad[row] != want[row], kw


# ---- generators -------------------------------------------------------------------------------------------------------

def test_generators(oracle):
    t = oracle.gen_trits(1, 200000)
    frac = [(t == v).mean() for v in (-1, 0, 1)]
    assert abs(frac[0] - 0.35) < 0.01 and abs(frac[1] - 0.30) < 0.01 and abs(frac[2] - 0.35) < 0.01
    a = oracle.gen_i8(2, 100000, -127, 127)
    assert a.min() == -127 and a.max() == 127
    assert np.array_equal(oracle.gen_trits(1, 1000), oracle.gen_trits(1, 1000))


# ---- golden fixtures ------------------------------------------------------------------------------------------------

def test_golden_fixtures_reproduce(oracle):
    import os
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    names = [n for n in os.listdir(gdir) if n.startswith("gemv_") and n.endswith(".npz")]
    assert len(names) >= 4
    for name in names:
        z = np.load(os.path.join(gdir, name))
        rows, cols = (int(v) for v in z["shape"])
        t = oracle.unpack_matrix(z["planar"], rows, cols)
        assert np.array_equal(z["acc"].astype(np.int64), t.astype(np.int64) @ z["acts"].astype(np.int64))
        assert np.array_equal(oracle.gemv_lut_planar(z["planar"], rows, cols, z["acts"]), z["acc"])
        y = oracle.epilogue_f32(z["acc"], float(z["weight_scale"]), float(z["act_scale"]))
        assert np.array_equal(y.view(np.uint32), z["y"].view(np.uint32))
    z = np.load(os.path.join(gdir, "config0_2560.npz"))
    t = oracle.gen_trits(int(z["trit_seed"]), (2560, 2560))
    a = oracle.gen_i8(int(z["act_seed"]), 2560, -127, 127)
    assert np.array_equal(z["acc"].astype(np.int64), t.astype(np.int64) @ a.astype(np.int64))
