"""Pins the oracle's GGUF ternary decoders (oracle/gguf_oracle.c) without restating them: encode -> decode round trips
over random matrices and the extremes (the reference's tq_decoders_roundtrip_encoder_output_for_every_trit_pattern,
quintrit-format/tests/gguf_decoder_tests.rs:569-584), the base-3 arithmetic of TQ1_0's bytes for every 5-trit value,
I2_S's bit planes for single trits, the ggml dequantizer layouts on the reference test's fixed byte pattern
(gguf_decoder_tests.rs:431-495), and Q2_0's rejection of code 3 (decoders/q2_0.rs:34-55)."""
import numpy as np
import pytest


def pseudo_trits(n: int, seed: int) -> np.ndarray:
    """xorshift64 trits, the reference test's generator (gguf_decoder_tests.rs:546-558)."""
    s = (seed | 1) & 0xFFFFFFFFFFFFFFFF
    out = np.empty(n, np.int8)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        out[i] = s % 3 - 1
    return out


@pytest.mark.parametrize("ty", [34, 35])
def test_tq_round_trips_and_extremes(oracle, ty):
    for rows, cols in [(1, 256), (4, 256), (3, 512), (32, 1024)]:
        t = pseudo_trits(rows * cols, 77 + rows)
        assert np.array_equal(oracle.tq_unpack(ty, oracle.tq_pack(ty, t), t.size), t)
    for v in (-1, 0, 1):
        t = np.full(256, v, np.int8)
        assert np.array_equal(oracle.tq_unpack(ty, oracle.tq_pack(ty, t), 256), t)
    # block sizes: 54 and 66 bytes per 256 weights, the f16 scale in the last two
    data = oracle.tq_pack(ty, np.zeros(512, np.int8), 0x3C00)
    bb = 54 if ty == 34 else 66
    assert data.size == 2 * bb and data[bb - 2] == 0x00 and data[bb - 1] == 0x3C


def test_tq1_0_bytes_are_base3_fractions_for_every_value():
    """TQ1_0 stores q in [0, 243) as ceil(q * 256 / 243); digit n of the byte is the n-th base-3 digit of q, most
    significant first, for all 243 values (every 5-trit pattern of a qs byte)."""
    from oracle import oracle as o
    trits = np.zeros((243, 256), np.int8)
    for q in range(243):
        digits = [(q // 3 ** (4 - n)) % 3 - 1 for n in range(5)]  # most significant first
        for n in range(5):
            trits[q, 32 * n + 5] = digits[n]  # element 32 n + m of qs byte m = 5
    data = o.tq_pack(34, trits.reshape(-1))
    for q in range(243):
        assert data[q * 54 + 5] == (q * 256 + 242) // 243
    assert np.array_equal(o.tq_unpack(34, data, trits.size), trits.reshape(-1))


def test_i2s_bit_planes_for_single_trits(oracle):
    """I2_S (decoders/i2_s.rs:18-42): trit j of a 128-trit block sits in byte j % 32 at bits 6 - 2 (j / 32), codes 0, 1,
    2 for -1, 0, +1; code 3 decodes to 0."""
    for j in (0, 31, 32, 77, 127):
        for v, code in ((-1, 0), (1, 2)):
            t = np.zeros((1, 256), np.int8)
            t[0, 128 + j] = v
            packed = oracle.i2s_pack(t)
            want = np.full(64, 0x55, np.uint8)
            sh = 6 - 2 * (j // 32)
            want[32 + j % 32] = (0x55 & ~(3 << sh)) | (code << sh)
            assert np.array_equal(packed, want), (j, v)
            assert np.array_equal(oracle.i2s_unpack(packed, 1, 256), t)
    three = np.full(32, 0xFF, np.uint8)
    assert np.array_equal(oracle.i2s_unpack(three, 1, 128), np.zeros((1, 128), np.int8))
    t = pseudo_trits(5 * 384, 9).reshape(5, 384)
    assert np.array_equal(oracle.i2s_unpack(oracle.i2s_pack(t), 5, 384), t)


def pattern_block(n: int) -> np.ndarray:
    return np.array([(i * 73 + 29) % 251 for i in range(n)], np.uint8)


def test_tq_layouts_on_the_reference_test_pattern(oracle):
    """The reference test's fixed bytes through the ggml dequantizer layouts it restates: TQ2_0 element 128 g + 32 l + m
    from bits 2 l of byte 32 g + m (gguf_decoder_tests.rs:431-441); TQ1_0 digits of qs[m] at 32 n + m, of qs[32 + m]
    at 160 + 16 n + m, of qh[j] at 240 + 4 n + j (gguf_decoder_tests.rs:445-471)."""
    b = pattern_block(66)
    got = oracle.tq_unpack(35, b, 256)
    code = lambda c: {0: -1, 2: 1}.get(int(c), 0)
    for g in range(2):
        for l in range(4):
            for m in range(32):
                assert got[128 * g + 32 * l + m] == code((b[32 * g + m] >> (2 * l)) & 3)
    b = pattern_block(54)
    got = oracle.tq_unpack(34, b, 256)
    dig = lambda byte, n: (((int(byte) * 3 ** n) & 255) * 3 >> 8) - 1
    for n in range(5):
        for m in range(32):
            assert got[32 * n + m] == dig(b[m], n)
        for m in range(16):
            assert got[160 + 16 * n + m] == dig(b[32 + m], n)
    for n in range(4):
        for j in range(4):
            assert got[240 + 4 * n + j] == dig(b[48 + j], n)


@pytest.mark.parametrize("block_size", [64, 128])
def test_q2_0_codes_scales_and_code3(oracle, block_size):
    rows, cols = 3, 256
    rng = np.random.default_rng(block_size)
    t = rng.integers(-1, 2, (rows, cols)).astype(np.int8)
    nb = rows * cols // block_size
    d = rng.integers(0, 0x7C00, nb).astype(np.uint16)
    blocks = []
    for blk in range(nb):
        w = t.reshape(-1)[blk * block_size:(blk + 1) * block_size] + 1
        q = (w[0::4] | (w[1::4] << 2) | (w[2::4] << 4) | (w[3::4] << 6)).astype(np.uint8)
        blocks.append(np.concatenate([np.array([d[blk] & 0xFF, d[blk] >> 8], np.uint8), q]))
    data = np.concatenate(blocks)
    got, scales = oracle.q2_0_unpack(data, rows, cols, block_size)
    assert np.array_equal(got, t)
    assert np.array_equal(scales, np.repeat(d, block_size // 64))
    bad = data.copy()
    bb = 2 + block_size // 4
    bad[bb + 2 + 3] |= 0xC0  # block 1, byte 3, weight 3: code 3
    with pytest.raises(ValueError, match=f"weight {block_size + 15} "):
        oracle.q2_0_unpack(bad, rows, cols, block_size)
