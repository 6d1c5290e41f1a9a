"""The AVX-512 transcription of the reference's production CPU GEMV (oracle/cpu_avx512.c), which bench.py times as the
CPU baseline: it must equal the brute-force int64 product on every shape before its timing means anything
(the reference's own ground truth, quintrit-core/tests/kernel_tests.rs:59-64). Skipped on hosts without AVX-512 VBMI.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def avx(oracle):
    if not oracle.cpu_avx512_supported():
        pytest.skip("no AVX-512 F/BW/VBMI on this host")
    return oracle


@pytest.mark.parametrize("rows,cols", [(64, 1), (64, 5), (64, 161), (128, 320), (192, 2560), (64, 3072),
                                        (256, 6912), (64, 23040)])
@pytest.mark.parametrize("threads", [1, 3])
def test_equals_bruteforce(avx, rows, cols, threads):
    o = avx
    rng = np.random.default_rng(rows * 7 + cols)
    t = o.gen_trits(int(rng.integers(1 << 30)), (rows, cols))
    a = o.gen_i8(int(rng.integers(1 << 30)), cols, -128, 127)
    got = o.gemv_avx512(o.tile64(o.pack_matrix(t), rows, cols), a, rows, cols, threads)
    np.testing.assert_array_equal(got.astype(np.int64), o.gemv_bruteforce(t, a))


@pytest.mark.parametrize("rows", [(192, 64, 64), (320, 128), (64,), (64, 64, 64, 64, 64)])
@pytest.mark.parametrize("threads", [1, 2, 3, 7])
def test_group_equals_bruteforce(avx, rows, threads):
    """The engine's projection group (one table build, the blocks of all matrices shared out over the threads, as
    forward_linear_triple / forward_linear_pair run them): every matrix equals its brute-force product, whichever
    thread's share crosses which matrix boundary."""
    o = avx
    cols = 3072
    rng = np.random.default_rng(sum(rows) + threads)
    a = o.gen_i8(int(rng.integers(1 << 30)), cols, -128, 127)
    ts = [o.gen_trits(int(rng.integers(1 << 30)), (r, cols)) for r in rows]
    got = o.gemv_group_avx512([o.tile64(o.pack_matrix(t), r, cols) for t, r in zip(ts, rows)], list(rows), a, cols,
                              threads)
    for g, t in zip(got, ts):
        np.testing.assert_array_equal(g.astype(np.int64), o.gemv_bruteforce(t, a))


@pytest.mark.parametrize("w,x", [(1, 127), (-1, 127), (1, -128), (-1, -128), (0, -128)])
def test_extreme_magnitudes(avx, w, x):
    """All weights one trit, all activations one extreme value: the int8 and int16 partial sums must not wrap."""
    o = avx
    rows, cols = 64, 23040
    t = np.full((rows, cols), w, np.int8)
    a = np.full(cols, x, np.int8)
    got = o.gemv_avx512(o.tile64(o.pack_matrix(t), rows, cols), a, rows, cols, 2)
    np.testing.assert_array_equal(got.astype(np.int64), np.full(rows, w * x * cols, np.int64))


def test_tile64_layout(avx):
    """transform_weights_lut_64 (avx512.rs:53-78): block b, tile column byte c, row r at b*64*tbr + c*64 + r % 64."""
    o = avx
    rows, cols = 128, 170
    t = o.gen_trits(5, (rows, cols))
    planar = o.pack_matrix(t)
    tiled = o.tile64(planar, rows, cols)
    tbr = o.tile_row_bytes(cols)
    rows_tiles = o.tile_rows(planar, rows, cols)
    for r in (0, 1, 63, 64, 127):
        for c in range(tbr):
            assert tiled[(r // 64) * 64 * tbr + c * 64 + r % 64] == rows_tiles[r, c]
