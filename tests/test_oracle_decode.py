"""Pins the decode-step oracle (oracle/decode_oracle.c) with checks that do not retype its code.

Sources of truth, in order of strength:
- the reference's own test vectors and models: the quantizer's known answers (quintrit-runtime/src/ops.rs:1968-1991),
  `dot_f16_model`, the portable statement of ggml_vec_dot_f16's operation order that the reference asserts its kernels
  equal bit for bit (ops.rs:2008-2060), and `ggml_vec_dot_bf16_scalar`, the reference's portable definition of the
  bf16 dot (ops.rs:686-713);
- the rounding semantics the reference's code states (FMA in the vector body of ggml_vec_mad_f16, separate roundings in
  its tail, ops.rs:1254-1300; round-to-nearest-even conversions, ops.rs:652-665) checked element by element with numpy;
- float64 restatements of the mathematics with tolerances, chosen so that a wrong index, sign, pairing or dropped term
  fails (RoPE, attention, the model forward, with a negative control that shows the tolerance is tight enough).
CPU only: no GPU is needed.
"""
from __future__ import annotations

import numpy as np
import pytest


def xorshift(seed: int):
    """test_rng of ops.rs:2036-2044 (64-bit xorshift 13/7/17)."""
    s = seed & 0xFFFFFFFFFFFFFFFF

    def nxt() -> int:
        nonlocal s
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        return s
    return nxt


def f16(v) -> np.ndarray:
    """f32 -> f16 bits with round to nearest even (the F16C conversion the reference uses)."""
    with np.errstate(over="ignore"):
        return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def h2f(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def bf2f(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint32) << 16).astype(np.uint32).view(np.float32)


# ---- quantizer: the reference's known answers -------------------------------------------------------------------------

def test_quantize_reference_known_answers(oracle):
    """ops.rs:1968-1991: [0.5, -1, 0.25, 1, -0.001] -> 127 / [64, -127, 32, 127, 0]; levels 63 -> [32, -63, 16, 63];
    all zeros -> scale 0 and zero codes."""
    q, s = oracle.quantize_i8(np.array([0.5, -1.0, 0.25, 1.0, -0.001], np.float32))
    assert s == np.float32(127.0) and list(q) == [64, -127, 32, 127, 0]
    q, s = oracle.quantize_i8(np.array([0.5, -1.0, 0.25, 1.0], np.float32), 63.0)
    assert s == np.float32(63.0) and list(q) == [32, -63, 16, 63]
    q, s = oracle.quantize_i8(np.zeros(8, np.float32))
    assert s == 0.0 and not q.any()


# ---- f16 / bf16 dot products --------------------------------------------------------------------------------------------

def dot_f16_model(x: np.ndarray, y: np.ndarray) -> np.float32:
    """The reference test's `dot_f16_model` (ops.rs:2008-2034): 4 accumulators of 8 lanes fed by fused multiply-adds
    over every 32 values, (a0 + a2) + (a1 + a3) per lane, then l + (l + 4) and a pairwise sum; the tail adds x * y.
    A product of two f16 values is exact in f32, so each fused multiply-add equals a multiply then an add."""
    fx, fy = h2f(x), h2f(y)
    n = len(fx)
    np_ = n & ~31
    acc = np.zeros((4, 8), np.float32)
    for i in range(0, np_, 32):
        acc = acc + fx[i:i + 32].reshape(4, 8) * fy[i:i + 32].reshape(4, 8)
    red = (acc[0] + acc[2]) + (acc[1] + acc[3])
    t0 = red[:4] + red[4:]
    s = (t0[0] + t0[1]) + (t0[2] + t0[3])
    for i in range(np_, n):
        s = np.float32(s + fx[i] * fy[i])
    return np.float32(s)


def test_dot_f16_equals_the_reference_model_bit_for_bit(oracle):
    """The reference asserts ggml_vec_dot_f16 == dot_f16_model at these lengths with this generator (ops.rs:2046-2061)."""
    nxt = xorshift(0x1234_5678_9ABC_DEF1)
    for n in (1, 7, 31, 32, 33, 64, 100, 256, 3072, 3079):
        for _ in range(20):
            x = f16([(np.float32(nxt() % 20001) - np.float32(10000.0)) * np.float32(1e-3) for _ in range(n)])
            y = f16([(np.float32(nxt() % 2001) - np.float32(1000.0)) * np.float32(1e-3) for _ in range(n)])
            got = np.float32(oracle.ggml_dot_f16(x, y))
            assert got.view(np.uint32) == dot_f16_model(x, y).view(np.uint32), n
    # half-precision special values: subnormals, the largest finite value, signed zeros (ops.rs:2057-2060)
    x = np.array([0x0001, 0x03FF, 0x7BFF, 0x8000, 0x0000, 0xFBFF, 0x0400, 0x3C00], np.uint16)
    y = np.array([0x3C00, 0x3C00, 0x0400, 0x3C00, 0x3C00, 0x0400, 0x7800, 0xBC00], np.uint16)
    assert np.float32(oracle.ggml_dot_f16(x, y)).view(np.uint32) == dot_f16_model(x, y).view(np.uint32)


def dot_bf16_definition(x: np.ndarray, y: np.ndarray) -> np.float32:
    """ggml_vec_dot_bf16_scalar (ops.rs:686-713), the reference's portable definition: acc + x * y rounded separately
    (a bf16 product is exact in f32), (a0 + a2) + (a1 + a3), the pairs (l4 + l0) ..., then the tail in double."""
    fx, fy = bf2f(x), bf2f(y)
    n = len(fx)
    acc = np.zeros((4, 8), np.float32)
    i = 0
    while i + 32 <= n:
        acc = acc + fx[i:i + 32].reshape(4, 8) * fy[i:i + 32].reshape(4, 8)
        i += 32
    a = (acc[0] + acc[2]) + (acc[1] + acc[3])
    g = a[4:] + a[:4]
    s = float((g[0] + g[2]) + (g[1] + g[3]))
    for k in range(i, n):
        s += float(fx[k] * fy[k])
    return np.float32(s)


def test_dot_bf16_equals_the_reference_definition(oracle):
    rng = np.random.default_rng(5)
    for n in (1, 31, 32, 33, 95, 2560, 2561, 4096):
        for _ in range(10):
            x = oracle_bf16(oracle, rng.standard_normal(n).astype(np.float32))
            y = oracle_bf16(oracle, (0.02 * rng.standard_normal(n)).astype(np.float32))
            got = np.float32(oracle.ggml_dot_bf16(x, y))
            assert got.view(np.uint32) == dot_bf16_definition(x, y).view(np.uint32), n


def oracle_bf16(oracle, v: np.ndarray) -> np.ndarray:
    return np.array([oracle.f32_to_bf16(float(e)) for e in v], np.uint16)


def test_bf16_conversions_match_torch(oracle):
    """f32 -> bf16 round to nearest even (ops.rs:658-665) equals torch's conversion; bf16 -> f32 is a shift."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 2000),
                        np.array([0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32)])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle_bf16(oracle, v)
    assert np.array_equal(got, want)
    for h in (0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F7F, 0x0001, 0x7F80):
        assert np.float32(oracle.bf16_to_f32(h)).view(np.uint32) == np.uint32(h << 16)


def test_f16_conversions_every_half(oracle):
    """Every f16 bit pattern widens exactly; f32 -> f16 rounds to nearest even (the F16C conversions, ops.rs:914-955)."""
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = hs.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(h)) for h in hs[::7]], np.float32)
    ok = (got.view(np.uint32) == want[::7].view(np.uint32)) | (np.isnan(got) & np.isnan(want[::7]))
    assert ok.all()
    rng = np.random.default_rng(8)
    v = (rng.standard_normal(5000) * 2.0 ** rng.integers(-28, 17, 5000)).astype(np.float32)
    got = np.array([oracle.f32_to_f16_bits(float(e)) for e in v], np.uint16)
    assert np.array_equal(got, f16(v))


# ---- f16 vector mad / scale ------------------------------------------------------------------------------------------------

def test_vec_mad_f16_rounding_semantics(oracle):
    """ggml_vec_mad_f16 (ops.rs:1254-1300, AVX2 path): the first n & ~31 values get f16(fma(x, v, y)), the tail
    f16(y + f32(x * v)). The fused result is computed here in float64 and kept only where that sum is exact (then one
    rounding to f32 is the FMA's)."""
    rng = np.random.default_rng(9)
    checked = 0
    for n in (31, 32, 64, 77, 128, 293):
        for _ in range(20):
            y = f16(rng.standard_normal(n).astype(np.float32) * 4)
            x = f16(rng.standard_normal(n).astype(np.float32) * 4)
            v = np.float32(rng.standard_normal() * 3)
            got = oracle.vec_mad_f16(y, x, float(v))
            fx, fy = h2f(x).astype(np.float64), h2f(y).astype(np.float64)
            p = fx * np.float64(v)             # exact: 11 x 24 significant bits
            s = p + fy
            exact = (s - p) == fy              # no rounding in the float64 sum
            body = f16(s.astype(np.float32))
            tail = f16(h2f(y) + h2f(x) * v)
            np_ = n & ~31
            want = np.concatenate([body[:np_], tail[np_:]])
            mask = np.concatenate([exact[:np_], np.ones(n - np_, bool)])
            assert np.array_equal(got[mask], want[mask]), n
            checked += int(mask.sum())
    assert checked > 10000


def _fused_unfused_split(rng, count):
    """f16 (x, y) pairs and an f32 v for which f16(fma(x, v, y)) and f16(y + f32(x * v)) differ: drawn at random and
    kept when the float64 sum x v + y is exact (so its rounding to f32 is the FMA's) and the two f16 results differ."""
    xs, ys, vs = [], [], []
    while len(xs) < count:
        x = f16(rng.standard_normal(4096).astype(np.float32) * 4)
        y = f16(rng.standard_normal(4096).astype(np.float32) * 4)
        v = (rng.standard_normal(4096) * 3).astype(np.float32)
        fx, fy = h2f(x).astype(np.float64), h2f(y).astype(np.float64)
        p = fx * v.astype(np.float64)
        s = p + fy
        fused = f16(s.astype(np.float32))
        unfused = f16(h2f(y) + (h2f(x) * v).astype(np.float32))
        keep = ((s - p) == fy) & (fused != unfused)
        xs += list(x[keep])
        ys += list(y[keep])
        vs += list(v[keep])
    return np.array(xs[:count], np.uint16), np.array(ys[:count], np.uint16), np.array(vs[:count], np.float32)


def test_vec_mad_f16_tail_is_unfused(oracle):
    """The n % 32 tail of ggml_vec_mad_f16 (ops.rs:1282-1287) is f32_to_f16(fy + fx * v): a multiply rounded to f32,
    then the add. Every tail element here is one where that differs from the fused f16(fma(x, v, y)) of the vector body,
    so an oracle that fuses the tail fails on all of them; the same pairs placed in the body must come out fused."""
    rng = np.random.default_rng(91)
    x, y, v = _fused_unfused_split(rng, 600)
    assert x.size == 600
    for i in range(0, 600, 31):  # one shared v per call: the pairs with that v only
        vi = v[i]
        sel = v == vi
        xt, yt = x[sel][:31], y[sel][:31]
        n = 32 + xt.size
        xb = f16(rng.standard_normal(32).astype(np.float32))
        yb = f16(rng.standard_normal(32).astype(np.float32))
        got = oracle.vec_mad_f16(np.concatenate([yb, yt]), np.concatenate([xb, xt]), float(vi))
        tail_want = f16(h2f(yt) + (h2f(xt) * vi).astype(np.float32))
        assert np.array_equal(got[32:n], tail_want)
    # the same pairs in the vector body: the fused rounding
    for k in range(0, 576, 32):
        for j in range(32):
            xx = np.full(32, x[k + j], np.uint16)
            yy = np.full(32, y[k + j], np.uint16)
            got = oracle.vec_mad_f16(yy, xx, float(v[k + j]))
            s = h2f(xx[:1]).astype(np.float64) * np.float64(v[k + j]) + h2f(yy[:1]).astype(np.float64)
            assert got[0] == f16(s.astype(np.float32))[0]
            assert got[0] != f16(h2f(yy[:1]) + (h2f(xx[:1]) * v[k + j]).astype(np.float32))[0]


def test_vec_scale_f16(oracle):
    """ggml_vec_scale_f16 (ops.rs:1304-1345): y = f16(f32(y) * v)."""
    rng = np.random.default_rng(10)
    for n in (1, 32, 293):
        y = f16(rng.standard_normal(n).astype(np.float32) * 4)
        v = np.float32(rng.uniform(0, 1))
        assert np.array_equal(oracle.vec_scale_f16(y, float(v)), f16(h2f(y) * v))


# ---- RoPE ---------------------------------------------------------------------------------------------------------------------

def test_rope_cache_recurrence(oracle):
    """rope_cache (ops.rs:121-140) with attn_factor 1 and no YaRN: theta_0 = pos, theta_{i+1} = theta_i * base^(-2/n)
    in f32; cache[2i] = cos(theta_i), cache[2i+1] = sin(theta_i). Position 0 is the identity."""
    c0 = oracle.rope_cache(0, 128, 500000.0)
    assert np.array_equal(c0[0::2], np.ones(64, np.float32)) and np.array_equal(c0[1::2], np.zeros(64, np.float32))
    scale = np.float32(np.float32(500000.0) ** np.float32(-2.0 / 128))
    for pos in (1, 2, 17, 319, 4095):
        c = oracle.rope_cache(pos, 128, 500000.0)
        theta = np.empty(64, np.float32)
        t = np.float32(pos)
        for i in range(64):
            theta[i] = t
            t = np.float32(t * scale)
        # the host libm's cosf/sinf against float64: within 2 f32 ulps
        assert np.allclose(c[0::2], np.cos(theta.astype(np.float64)), rtol=0, atol=2.5e-7)
        assert np.allclose(c[1::2], np.sin(theta.astype(np.float64)), rtol=0, atol=2.5e-7)


def test_rope_neox_pairs_and_signs(oracle):
    """NEOX pairing (ops.rs:199-221, offset n_dims / 2): pair i rotates (x[i], x[i + half]); with cos 0 and sin 1 on one
    pair the rotation is exact: (x0, x1) -> (-x1, x0); every other pair (cos 1, sin 0) is unchanged."""
    heads, hd = 3, 128
    rng = np.random.default_rng(11)
    x = rng.standard_normal(heads * hd).astype(np.float32)
    for k in (0, 5, 63):
        cache = np.zeros(hd, np.float32)
        cache[0::2] = 1.0
        cache[2 * k], cache[2 * k + 1] = 0.0, 1.0
        got = oracle.rope_neox(x, heads, hd, cache)
        want = x.copy().reshape(heads, hd)
        want[:, k], want[:, k + 64] = -x.reshape(heads, hd)[:, k + 64], x.reshape(heads, hd)[:, k]
        assert np.array_equal(got.reshape(heads, hd), want)
    cache = oracle.rope_cache(77, hd, 500000.0)
    got = oracle.rope_neox(x, heads, hd, cache).reshape(heads, hd).astype(np.float64)
    c, s = cache[0::2].astype(np.float64), cache[1::2].astype(np.float64)
    xx = x.reshape(heads, hd).astype(np.float64)
    assert np.allclose(got[:, :64], xx[:, :64] * c - xx[:, 64:] * s, rtol=0, atol=1e-6)
    assert np.allclose(got[:, 64:], xx[:, :64] * s + xx[:, 64:] * c, rtol=0, atol=1e-6)


def test_rope_normal_pairs_and_signs(oracle):
    """Normal pairing (ops.rs:199-221, offset 1, stride 2; Falcon3's RopeMode::Normal): pair i rotates (x[2i], x[2i+1]);
    a one-hot (cos 0, sin 1) pair maps (x0, x1) -> (-x1, x0) exactly and leaves every other pair unchanged."""
    heads, hd = 2, 256
    rng = np.random.default_rng(12)
    x = rng.standard_normal(heads * hd).astype(np.float32)
    for k in (0, 7, 127):
        cache = np.zeros(hd, np.float32)
        cache[0::2] = 1.0
        cache[2 * k], cache[2 * k + 1] = 0.0, 1.0
        got = oracle.rope_normal(x, heads, hd, cache)
        want = x.copy().reshape(heads, hd)
        xx = x.reshape(heads, hd)
        want[:, 2 * k], want[:, 2 * k + 1] = -xx[:, 2 * k + 1], xx[:, 2 * k]
        assert np.array_equal(got.reshape(heads, hd), want)
    cache = oracle.rope_cache(123, hd, 100000.0)
    got = oracle.rope_normal(x, heads, hd, cache).reshape(heads, hd).astype(np.float64)
    c, s = cache[0::2].astype(np.float64), cache[1::2].astype(np.float64)
    xx = x.reshape(heads, hd).astype(np.float64)
    assert np.allclose(got[:, 0::2], xx[:, 0::2] * c - xx[:, 1::2] * s, rtol=0, atol=1e-6)
    assert np.allclose(got[:, 1::2], xx[:, 0::2] * s + xx[:, 1::2] * c, rtol=0, atol=1e-6)


# ---- SiLU / SwiGLU (Falcon3) -------------------------------------------------------------------------------------------------

def f32_ulp(v: np.ndarray) -> np.ndarray:
    return np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float32)).astype(np.float64)


def test_ggml_expf_error_bound_and_branches(oracle):
    """ggml_v_expf_avx2 (ops.rs:314-377) lane by lane: exp(0) = 1 exactly; over the normal range within 2 ulps of
    float64 exp (ggml states 1.45 + 0.5 ulp; measured 1.94), which a wrong constant, a dropped polynomial term or a
    swapped coefficient pair breaks by orders of magnitude; the scaled branch for results below 2^-126 within 2 units
    of 2^-149; 0 below and inf above the float range; NaN propagates. The reference's own test asks 3e-6 relative on
    [-40, 40] (algorithm_tests.rs:191-219)."""
    assert oracle.ggml_expf(0.0) == 1.0 and oracle.ggml_expf(-0.0) == 1.0
    rng = np.random.default_rng(31)
    x = np.concatenate([np.linspace(-87.3, 88.7, 400001, dtype=np.float32),
                        rng.uniform(-10, 10, 100000).astype(np.float32),
                        np.arange(-80, 80, dtype=np.float32) * np.float32(0.5)])
    got = oracle.ggml_expf_array(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(got - want) / f32_ulp(want)) <= 2.0
    sub = np.linspace(-103.9, -87.4, 20001, dtype=np.float32)
    g = oracle.ggml_expf_array(sub).astype(np.float64)
    assert np.max(np.abs(g - np.exp(sub.astype(np.float64)))) <= 2 * 2.0 ** -149
    edge = oracle.ggml_expf_array(np.array([88.73, 89.0, 200.0, np.inf, -104.0, -150.0, -np.inf, np.nan], np.float32))
    assert np.all(np.isinf(edge[:4])) and np.all(edge[:4] > 0)
    assert np.array_equal(edge[4:7], np.zeros(3, np.float32)) and np.isnan(edge[7])


def test_swiglu_blocks_and_tail(oracle):
    """swiglu (ops.rs:430-464): silu(g) * u within 4 ulps of float64 for every length (SiLU = x / (1 + exp(-x)) with
    the vector exponential on whole blocks of 8); the last n % 8 values take the libm exponential: a block result does
    not depend on the length (prefixes agree), and the tail equals v / (1 + expf(-v)) * u with the host expf."""
    rng = np.random.default_rng(4)
    for n in (7, 8, 33, 256, 23040):
        g = (rng.standard_normal(n) * 8).astype(np.float32)
        u = (rng.standard_normal(n) * 2).astype(np.float32)
        got = oracle.swiglu(g, u)
        gx, ux = g.astype(np.float64), u.astype(np.float64)
        want = gx / (1.0 + np.exp(-gx)) * ux
        assert np.all(np.abs(got - want) <= 4 * f32_ulp(want) + 1e-40), n
        n8 = n // 8 * 8
        if n8:
            assert np.array_equal(got[:n8], oracle.swiglu(g[:n8], u[:n8]))
        if n8 < n:
            t = g[n8:]
            den = np.float32(1.0) + oracle.expf(-t)
            assert np.array_equal(got[n8:], (t / den) * u[n8:])
    # the vector and libm exponentials differ in the last bit on many inputs, so the tail rule is observable
    t = rng.uniform(-10, 10, 4096).astype(np.float32)
    assert np.any(oracle.ggml_expf_array(t) != oracle.expf(t))


# ---- attention ------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("seq_len,max_ctx", [(1, 4096), (37, 4096), (300, 4096), (600, 4096), (1500, 2048), (600, 640)])
def test_attend_head_close_to_float64(oracle, seq_len, max_ctx):
    """attend_head (attention.rs:483-542), both the single online softmax and the 4-chunk split (padded length >= 512),
    against float64 softmax attention over the same f16 q, k, v. The FP16 value accumulator limits the agreement."""
    hd = 128
    rng = np.random.default_rng(seq_len)
    q = f16(rng.standard_normal(hd).astype(np.float32))
    k = f16(rng.standard_normal((seq_len, hd)).astype(np.float32))
    v = f16(rng.standard_normal((seq_len, hd)).astype(np.float32))
    scale = 1.0 / np.sqrt(hd)
    got = oracle.attend_head(q, k, v, seq_len, max_ctx, float(np.float32(scale))).astype(np.float64)
    sc = h2f(k).astype(np.float64) @ h2f(q).astype(np.float64) * np.float64(np.float32(scale))
    p = np.exp(sc - sc.max())
    want = (p / p.sum()) @ h2f(v).astype(np.float64)
    assert np.max(np.abs(got - want)) < 2e-3 * max(1.0, np.max(np.abs(want)))


# Closed forms of attend_head where every softmax weight is exactly 0 or 1. The query is e0 (f16 1.0 in coordinate 0)
# and each key carries a level of 0 or 60000 in coordinate 0, so a score is 0 or 60000 * scale (~5300); exp(0) = 1 and
# exp(-5300) = 0 in f32. Within an online-softmax range the positions from the first occurrence of the range's highest
# level on, at that level, are summed with weight 1 into the FP16 accumulator (each step f16(f32(acc) + f32(v)), which
# is what f16(fma(v, 1, acc)) and the tail's f16(acc + f32(v * 1)) both are), earlier ones are wiped by a factor 0, later
# lower ones are added with weight 0. Chunks whose highest level is below the global one drop out of the combine
# (factor 0); the others are added in chunk order in f32. So the output is fixed by sums a reader can do by hand, and
# these sums expose the padded length, the split threshold, the chunk size, the accumulator precision and the combine
# order (attention.rs:436-468,483-542).

SPIKE = 60000.0


def attn_closed_form(levels, v, seq_len, max_ctx, *, chunk_from_seq=False, f16_acc=True, pad=True, n_chunks=4,
                     reverse=False):
    hd = v.shape[1]
    n_kv = max(-(-seq_len // 256) * 256, 256) if pad else seq_len
    n_kv = min(n_kv, max_ctx)

    def run(lo, hi):
        lv = levels[lo:hi]
        m = lv.max()
        first = lo + int(np.argmax(lv == m))
        acc = np.zeros(hd, np.float32)
        count = 0
        for p in range(first, hi):
            if levels[p] == m:
                acc = acc + h2f(v[p])
                if f16_acc:
                    acc = h2f(f16(acc))
                count += 1
        return m, acc, count

    if n_kv < 512:
        _, acc, s = run(0, seq_len)
        return acc * (np.float32(1) / np.float32(s))
    chunk = -(-(seq_len if chunk_from_seq else n_kv) // n_chunks)
    parts = []
    for c in range(n_chunks):
        lo, hi = c * chunk, min(c * chunk + chunk, n_kv, seq_len)
        if lo < hi:
            parts.append(run(lo, hi))
    if reverse:
        parts = parts[::-1]
    top = max(p[0] for p in parts)
    acc = np.zeros(hd, np.float32)
    s = np.float32(0)
    for m, a, n in parts:
        if m == top:
            acc = acc + a
            s = np.float32(s + n)
    return acc * (np.float32(1) / s)


def attn_structured_inputs(seq_len, hd, spikes, seed):
    """q = e0; keys: level 0 or SPIKE in coordinate 0, random elsewhere. Values (none of them -0):
    column 0 is 2048 at position 0 and 1.0 elsewhere (2048 + 1 rounds back to 2048 in f16, so an FP16 chain absorbs
    every 1.0 after it while a new chunk counts them exactly); column 1 is 32768 at position 0 and 2^-9 at every 37th
    position (absorbed in f16 inside a chunk; in the f32 combine 32768 + 2^-9 is a tie that rounds to 32768, so the
    combine order shows); the other columns are random magnitudes in [0.25, 4) of both signs."""
    rng = np.random.default_rng(seed)
    levels = np.zeros(seq_len)
    if spikes:
        levels[np.arange(seq_len) % 97 == 13] = SPIKE
    q = np.zeros(hd, np.float32)
    q[0] = 1.0
    k = rng.uniform(-2, 2, (seq_len, hd)).astype(np.float32)
    k[:, 0] = levels
    vv = rng.uniform(0.25, 4, (seq_len, hd)) * rng.choice([-1.0, 1.0], (seq_len, hd))
    vv[:, 0] = 1.0
    vv[0, 0] = 2048.0
    vv[:, 1] = 0.0
    vv[::37, 1] = 2.0 ** -9
    vv[0, 1] = 32768.0
    return f16(q), f16(k), f16(vv.astype(np.float32)), levels


ATTN_CASES = [(200, 4096), (256, 4096), (257, 4096), (300, 400), (513, 4096), (600, 4096), (600, 640), (1500, 2048)]


@pytest.mark.parametrize("spikes", [False, True])
@pytest.mark.parametrize("seq_len,max_ctx", ATTN_CASES)
def test_attend_head_closed_form(oracle, seq_len, max_ctx, spikes):
    """attend_head equals the 0/1-weight closed form bit for bit: KV padded to a multiple of 256 (at least 256, at most
    the cache length), one online softmax below a padded length of 512, else 4 chunks of ceil(n_kv / 4) positions, FP16
    accumulators per chunk, an f32 combine in chunk order (attention.rs:483-542). With equal keys (no spikes) the
    single-softmax output is the plain f16 sequential sum of V divided by n."""
    hd = 40  # 32 values in ggml_vec_mad_f16's vector body, 8 in its tail
    q, k, v, levels = attn_structured_inputs(seq_len, hd, spikes, seq_len)
    scale = np.float32(1.0 / np.sqrt(128.0))
    got = oracle.attend_head(q, k, v, seq_len, max_ctx, float(scale))
    want = attn_closed_form(levels, v, seq_len, max_ctx)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if not spikes and seq_len <= 256:
        seqsum = np.zeros(hd, np.uint16)
        for p in range(seq_len):
            seqsum = f16(h2f(seqsum) + h2f(v[p]))
        plain = h2f(seqsum) * (np.float32(1) / np.float32(seq_len))
        assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))
        assert h2f(seqsum)[0] == 2048.0  # every 1.0 absorbed by the f16 chain


def test_attend_head_closed_form_negative_controls(oracle):
    """The closed-form check rejects each plausible mistake: a chunk size from seq_len instead of the padded n_kv, an
    f32 value accumulator, no KV padding (split decided by seq_len), 8 chunks, and a reversed combine. For each mutant
    some case gives an output different from the oracle's, so an oracle that made that mistake would fail
    test_attend_head_closed_form."""
    hd = 40
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    mutants = dict(chunk_from_seq=dict(chunk_from_seq=True), f32_acc=dict(f16_acc=False), no_pad=dict(pad=False),
                   eight_chunks=dict(n_chunks=8), reverse=dict(reverse=True))
    caught = {name: [] for name in mutants}
    for spikes in (False, True):
        for seq_len, max_ctx in ATTN_CASES:
            q, k, v, levels = attn_structured_inputs(seq_len, hd, spikes, seq_len)
            got = oracle.attend_head(q, k, v, seq_len, max_ctx, scale)
            for name, kw in mutants.items():
                bad = attn_closed_form(levels, v, seq_len, max_ctx, **kw)
                if not np.array_equal(got.view(np.uint32), bad.view(np.uint32)):
                    caught[name].append((seq_len, max_ctx, spikes))
    for name, where in caught.items():
        assert where, f"the closed-form check does not see the mutant {name}"
    # the chunk-size mistake at the case the review named: seq 600 pads to 768, so chunks are 192 positions, not 150
    assert (600, 4096, False) in caught["chunk_from_seq"]
    assert (600, 4096, False) in caught["f32_acc"]


# ---- the model forward against a float64 model written from model.rs / attention.rs -------------------------------------

TINY = dict(n_layers=2, hidden=160, n_heads=4, n_kv_heads=2, head_dim=32, ffn=320, vocab=300, max_ctx=64)


def rms64(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def quant64(y):
    """quantize_activations_int8_with_range (ops.rs:241-267) in float64: s = 127 / max|y|, round half away from zero."""
    m = np.max(np.abs(y))
    if m == 0:
        return np.zeros_like(y), 0.0
    s = 127.0 / m
    q = np.clip(np.sign(y * s) * np.floor(np.abs(y * s) + 0.5), -128, 127)
    return q, s


def f64_forward(model, cfg, tokens, skip_subnorm=False, swap_rope=False):
    """model.rs:282-377, 64-203 and attention.rs:115-260 in float64: RMSNorm -> int8 -> ternary projection with
    out = acc * ws / as -> RoPE (NEOX, or Normal for Falcon3) -> GQA softmax attention -> [sub-norm] -> o -> residual;
    RMSNorm -> gate, up -> relu(gate)^2 * up or silu(gate) * up -> [sub-norm] -> down -> residual; final norm ->
    the head's type -> the head (tied bf16, or untied f16). swap_rope takes the other pairing (a negative control)."""
    import oracle.oracle as o
    L, H, F, hd = cfg.n_layers, cfg.hidden, cfg.ffn, cfg.head_dim
    nh, nkv = cfg.n_heads, cfg.n_kv_heads
    sub = not cfg.no_sub_norm
    normal = (cfg.rope_mode == o.ROPE_NORMAL) != swap_rope
    W = {}
    for l in range(L):
        for kind in range(7):
            rows, cols = model.projection_shape(kind)
            planar, ws = model.projection(l, kind)
            W[l, kind] = (o.unpack_matrix(planar, rows, cols).astype(np.float64), float(ws))
    norms = {(l, k): model.norm(l, k).astype(np.float64) for l in range(L) for k in range(4) if sub or k in (0, 2)}
    out_norm = model.norm(L, 0).astype(np.float64)
    to_f = h2f if cfg.emb_f16 else bf2f
    emb = to_f(model.embedding()).astype(np.float64)
    head = to_f(model.head()).astype(np.float64)
    eps = float(np.float32(cfg.rms_eps))

    def proj(l, kind, xn):
        qv, s = quant64(xn)
        w, ws = W[l, kind]
        return np.zeros(w.shape[0]) if s == 0 else (w @ qv) * (ws / s)

    def rope(x, heads, pos):
        x = x.reshape(heads, hd).copy()
        i = np.arange(hd // 2)
        th = pos * float(cfg.rope_theta) ** (-2.0 * i / hd)
        c, s = np.cos(th), np.sin(th)
        if normal:
            x0, x1 = x[:, 0::2].copy(), x[:, 1::2].copy()
            x[:, 0::2], x[:, 1::2] = x0 * c - x1 * s, x0 * s + x1 * c
        else:
            x0, x1 = x[:, :hd // 2].copy(), x[:, hd // 2:].copy()
            x[:, :hd // 2], x[:, hd // 2:] = x0 * c - x1 * s, x0 * s + x1 * c
        return x

    kc = [[] for _ in range(L)]
    vc = [[] for _ in range(L)]
    logits = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        for l in range(L):
            xn = rms64(x, norms[l, 0], eps)
            q = rope(proj(l, 0, xn), nh, pos)
            k = rope(proj(l, 1, xn), nkv, pos)
            v = proj(l, 2, xn).reshape(nkv, hd)
            kc[l].append(k)
            vc[l].append(v)
            K, V = np.stack(kc[l]), np.stack(vc[l])
            att = np.empty((nh, hd))
            for h in range(nh):
                kvh = h // (nh // nkv)
                sc = K[:, kvh] @ q[h] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ V[:, kvh]
            a = att.reshape(-1)
            xn = a if (skip_subnorm or not sub) else rms64(a, norms[l, 1], eps)
            x = x + proj(l, 3, xn)
            xn = rms64(x, norms[l, 2], eps)
            g, u = proj(l, 4, xn), proj(l, 5, xn)
            if cfg.act == o.ACT_SILU:
                inter = g / (1.0 + np.exp(-g)) * u
            else:
                inter = np.maximum(g, 0.0) ** 2 * u
            x = x + proj(l, 6, rms64(inter, norms[l, 3], eps) if sub else inter)
        xn = rms64(x, out_norm, eps).astype(np.float32)
        xb = (h2f(f16(xn)) if cfg.emb_f16 else bf2f(f16_to_bf16_bits(xn))).astype(np.float64)
        logits.append(head @ xb)
    return np.array(logits)


def f16_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_model_forward_close_to_float64_model(oracle):
    """Logits of the oracle's forward over 12 positions against the float64 model: the structure (residuals, norms and
    sub-norms, GQA head mapping, NEOX RoPE, relu^2 gating, tied head) must match; the difference that remains comes from
    f32 / f16 rounding and int8 codes that land on the other side of a rounding boundary. The negative control (the
    float64 model without the attention sub-norm) must miss the same tolerance."""
    cfg = oracle.ModelConfig(TINY["n_layers"], TINY["hidden"], TINY["n_heads"], TINY["n_kv_heads"], TINY["head_dim"],
                             TINY["ffn"], TINY["vocab"], TINY["max_ctx"], 1e-5, 500000.0)
    m = oracle.Model(cfg, 0x51DE)
    tokens = [int(t) for t in np.random.default_rng(3).integers(0, cfg.vocab, 12)]
    m.reset()
    got = np.array([m.forward(t, p)[1] for p, t in enumerate(tokens)], np.float64)
    want = f64_forward(m, cfg, tokens)
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    # Measured: at most 3.3 % of the largest logit per position; structural mistakes in the float64 model (another GQA
    # mapping, a dropped sub-norm or residual, NORMAL instead of NEOX pairing, SiLU instead of relu^2) give 57-190 %.
    err = np.max(np.abs(got - want) / scale)
    assert err < 0.06, err
    bad = f64_forward(m, cfg, tokens, skip_subnorm=True)
    assert np.max(np.abs(got - bad) / scale) > 0.3
    agree = np.mean(np.argmax(got, axis=1) == np.argmax(want, axis=1))
    assert agree >= 0.75
    m.close()


def test_rms_norm_follows_the_reference_text(oracle):
    """rms_norm_avx2 (ops.rs:61-96): each square rounded to f32, summed in order in f64, mean rounded to f32,
    inv = 1 / sqrt(mean + eps) in f32, out = (x * inv) * w in f32. np.cumsum accumulates in order, so its last element
    is the sequential sum."""
    rng = np.random.default_rng(23)
    for n in (1, 7, 2560, 3079, 6912):
        x = (rng.standard_normal(n) * np.exp(rng.uniform(-8, 3, n))).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        ss = np.cumsum((x * x).astype(np.float64))[-1]
        mean = np.float32(ss / n)
        inv = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(1e-5)))
        want = (x * inv) * w
        assert np.array_equal(oracle.rms_norm(x, w, 1e-5).view(np.uint32), want.view(np.uint32)), n


def test_falcon3_forward_close_to_float64_model(oracle):
    """The Falcon3 switches of the oracle's forward (SwiGLU, Normal RoPE, no sub-norms, f16 embedding, untied f16 head)
    against the float64 model with the same switches, over 12 positions (measured: 2.1 % of the largest logit). The
    negative control pairs RoPE the NEOX way (85 %) and must miss the same tolerance; ReLU^2 in place of SiLU gives
    62 %."""
    cfg = oracle.falcon3(2, 160, 4, 2, 32, 320, 300, 64, 1e-5, 10000.0)
    m = oracle.Model(cfg, 0xFA1C)
    assert m.norm(0, 1) is None and m.norm(0, 3) is None
    assert not np.array_equal(m.head(), m.embedding())
    tokens = [int(t) for t in np.random.default_rng(8).integers(0, cfg.vocab, 12)]
    m.reset()
    got = np.array([m.forward(t, p)[1] for p, t in enumerate(tokens)], np.float64)
    want = f64_forward(m, cfg, tokens)
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    err = np.max(np.abs(got - want) / scale)
    assert err < 0.06, err
    bad = f64_forward(m, cfg, tokens, swap_rope=True)
    assert np.max(np.abs(got - bad) / scale) > 0.3
    assert np.mean(np.argmax(got, axis=1) == np.argmax(want, axis=1)) >= 0.75
    m.close()
