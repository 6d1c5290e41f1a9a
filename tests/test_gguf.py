"""The GGUF reader and the host transcoder of libvelurex_hip (vx_gguf_*, quintrit_amd.gguf), on the CPU.

Mirrors the reference's format tests (quintrit-format/tests/gguf_decoder_tests.rs, hostile_files.rs): every metadata
type and the architecture accessors, typed tensor payloads, alignment, the I2_S trailing scale and the TQ block scales,
Q2_0 block-size detection, and hostile files (bad magic and versions, truncation at every length, counts and lengths
beyond the file, long keys, invalid UTF-8, deep arrays, bad alignment and offsets, overlapping payloads). The host
conversion to planar velurex bytes is compared with the oracle's decoders and packer."""
import os
import struct

import numpy as np
import pytest

from gguf_writer import ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, build

from quintrit_amd._lib import VxError
from quintrit_amd.gguf import GgufFile, ggml_to_planar


@pytest.fixture
def write(tmp_path):
    def w(name, data):
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        return str(p)
    return w


def f16bits(v):
    return np.array(v, np.float32).astype(np.float16).view(np.uint16)


def test_all_metadata_types_and_architecture_accessors(write):
    kvs = [("general.architecture", STR, "bitnet"), ("bitnet.context_length", U32, 4096),
           ("bitnet.embedding_length", U64, 2560), ("bitnet.block_count", I32, 30),
           ("bitnet.feed_forward_length", U32, 6912), ("bitnet.attention.head_count", U16, 20),
           ("bitnet.attention.head_count_kv", U8, 5), ("bitnet.attention.layer_norm_rms_epsilon", F32, 1e-5),
           ("bitnet.rope.freq_base", F64, 500000.0), ("bitnet.vocab_size", I64, 128256),
           ("x.i8", I8, -3), ("x.i16", I16, -300), ("x.bool", BOOL, 1), ("x.neg", I32, -1),
           ("tokenizer.ggml.tokens", ARR, ["a", "b", "ü"], STR),
           ("x.nested", ARR, [(U32, [1, 2]), (U32, [3])], ARR)]
    with GgufFile(write("meta", build(kvs, []))) as g:
        assert g.version == 3 and g.tensors == {}
        assert g.architecture() == "bitnet"
        assert (g.context_length(), g.embedding_length(), g.block_count()) == (4096, 2560, 30)
        assert (g.feed_forward_length(), g.head_count(), g.head_count_kv(), g.vocab_size()) == (6912, 20, 5, 128256)
        assert g.rms_norm_eps() == float(np.float32(1e-5)) and g.rope_freq_base() == 500000.0
        assert g.metadata["x.i8"] == -3 and g.metadata["x.i16"] == -300 and g.metadata["x.bool"] is True
        assert g.metadata["tokenizer.ggml.tokens"] == ["a", "b", "ü"]
        assert g.metadata["x.nested"] == [[1, 2], [3]]
        assert g.metadata_types["x.nested"] == (ARR, ARR)
        from quintrit_amd._lib import lib
        import ctypes
        v = ctypes.c_uint64()
        assert lib().vx_gguf_metadata_u64(g.handle, b"x.neg", ctypes.byref(v)) != 0  # negative is not unsigned
        assert lib().vx_gguf_metadata_u64(g.handle, b"nope", ctypes.byref(v)) == 9   # VX_ERR_NOT_FOUND
        n = ctypes.c_size_t()
        assert lib().vx_gguf_metadata_string(g.handle, b"general.architecture", None, 0, ctypes.byref(n)) == 4
        assert n.value == 6
    with GgufFile(write("noarch", build([("general.name", STR, "x")], []))) as g:
        assert g.architecture() is None and g.context_length() is None and g.rms_norm_eps() is None


def test_tensor_accessors_scale_and_alignment(write, oracle):
    f = np.array([1.5, -2.0, 0.25], np.float32)
    h = f16bits([1.0, -0.5])
    trits = np.random.default_rng(1).integers(-1, 2, (2, 128)).astype(np.int8)
    i2 = oracle.i2s_pack(trits)
    tensors = [("a.f32", [3], 0, f.tobytes()), ("b.f16", [2], 1, h.tobytes()),
               ("w.i2s", [128, 2], 36, i2.tobytes() + struct.pack("<f", 0.75))]
    for alignment in (32, 64):
        kvs = [] if alignment == 32 else [("general.alignment", U32, alignment)]
        with GgufFile(write(f"t{alignment}", build(kvs, tensors, alignment))) as g:
            assert g.data_start % alignment == 0
            assert np.array_equal(g.get_tensor_f32("a.f32"), f)
            assert np.array_equal(g.get_tensor_f16("b.f16"), h)
            assert g.get_tensor_f32("b.f16") is None and g.get_tensor_data("missing") is None
            t = g.tensors["w.i2s"]
            assert t.shape == (128, 2) and t.tensor_type == 36 and t.byte_len == 64 and t.type_name == "I2_S"
            assert np.array_equal(g.get_tensor_data("w.i2s"), i2)
            assert g.get_tensor_scale("w.i2s") == 0.75 and g.get_tensor_scale("a.f32") == 1.0
            assert g.unread_tensors() == []
            planar, rows, cols, scale = g.convert_planar("w.i2s")
            assert (rows, cols, scale) == (2, 128, 0.75)
            assert np.array_equal(planar, oracle.pack_matrix(trits).reshape(-1))


@pytest.mark.parametrize("ty", [34, 35, 36])
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 512), (2, 384), (7, 1280), (2, 23040)])
def test_host_conversion_matches_the_oracle(oracle, ty, rows, cols):
    """vx_ggml_to_planar == oracle decode -> oracle pack, including rows that are not whole TQ blocks (cols 384) and
    rows whose last 160-trit block is partial."""
    if ty == 36 and cols % 128:
        pytest.skip("I2_S needs cols % 128 == 0")
    if ty != 36 and rows * cols % 256:
        pytest.skip("TQ needs whole blocks")
    rng = np.random.default_rng(rows * 1000 + cols + ty)
    trits = rng.integers(-1, 2, (rows, cols)).astype(np.int8)
    data = oracle.i2s_pack(trits) if ty == 36 else oracle.tq_pack(ty, trits.reshape(-1))
    want_trits = oracle.i2s_unpack(data, rows, cols) if ty == 36 else oracle.tq_unpack(ty, data, rows * cols).reshape(rows, cols)
    assert np.array_equal(want_trits, trits)
    assert np.array_equal(ggml_to_planar(ty, data, rows, cols), oracle.pack_matrix(trits).reshape(-1))


def test_host_conversion_of_arbitrary_bytes(oracle):
    """Every payload byte is defined: I2_S and TQ2_0 code 3 reads as 0, TQ1_0 digits of any byte are in {-1, 0, 1}."""
    rng = np.random.default_rng(3)
    for ty, nbytes in ((36, 2 * 256 // 4), (35, 2 * 66), (34, 2 * 54)):
        data = rng.integers(0, 256, nbytes).astype(np.uint8)
        trits = oracle.i2s_unpack(data, 2, 256) if ty == 36 else oracle.tq_unpack(ty, data, 512).reshape(2, 256)
        assert np.array_equal(ggml_to_planar(ty, data, 2, 256), oracle.pack_matrix(trits).reshape(-1))


def test_conversion_errors():
    with pytest.raises(VxError, match="UNSUPPORTED"):
        ggml_to_planar(1, np.zeros(512, np.uint8), 1, 256)
    with pytest.raises(VxError, match="INVALID_SHAPE"):
        ggml_to_planar(36, np.zeros(512, np.uint8), 1, 100)
    with pytest.raises(VxError, match="BUFFER_TOO_SMALL"):
        ggml_to_planar(34, np.zeros(53, np.uint8), 1, 256)


def test_tq_block_scales(write, oracle):
    trits = np.random.default_rng(5).integers(-1, 2, 4 * 256).astype(np.int8)
    same = oracle.tq_pack(34, trits, 0x3800)
    differ = same.copy()
    differ[54 + 52] ^= 1  # the second block's scale
    tensors = [("same", [256, 4], 34, same.tobytes()), ("differ", [256, 4], 34, differ.tobytes()),
               ("tq2", [512, 2], 35, oracle.tq_pack(35, trits, 0xC000).tobytes())]
    with GgufFile(write("tq", build([], tensors))) as g:
        assert g.get_tensor_scale("same") == 0.5 and g.get_tensor_scale("tq2") == -2.0
        with pytest.raises(VxError, match="differing per-block scales"):
            g.get_tensor_scale("differ")
        with pytest.raises(VxError, match="FORMAT"):
            g.convert_planar("differ")
        planar, rows, cols, scale = g.convert_planar("tq2")
        assert (rows, cols, scale) == (2, 512, -2.0)
        assert np.array_equal(planar, oracle.pack_matrix(trits.reshape(2, 512)).reshape(-1))


def test_q2_0_block_size_from_the_layout(write):
    """gguf.rs:460-508: 18-byte blocks of 64 or 34-byte blocks of 128 weights, told apart by where the next tensor
    starts; tensors that cannot tell take the others' size; disagreeing tensors are rejected."""
    n = 4096
    t64 = ("q64", [n], 42, bytes(n // 64 * 18))
    t128 = ("q128", [n], 42, bytes(n // 128 * 34))
    f = ("f", [8], 0, bytes(32))
    with GgufFile(write("q64", build([], [t64, f]))) as g:
        assert g.tensors["q64"].block_size == 64 and g.tensors["q64"].byte_len == n // 64 * 18
        assert g.tensors["f"].block_size is None
    with GgufFile(write("q128", build([], [t128, f]))) as g:
        assert g.tensors["q128"].block_size == 128
    with pytest.raises(VxError, match="different block sizes"):
        GgufFile(write("mixed", build([], [t64, t128, f])))


def test_q2_0_block_detection_scales_with_many_tensors(write):
    """A file of many small Q2_0 tensors: the block size of each is read from the next tensor's start, found by a
    binary search over the sorted starts, so opening stays fast (a scan per tensor would be quadratic in their count)."""
    import time
    n_t = 40000
    tensors = [(f"q{i}", [64], 42, bytes(18)) for i in range(n_t)]
    path = write("many_q2", build([], tensors))
    t0 = time.perf_counter()
    with GgufFile(path) as g:
        assert len(g.tensors) == n_t
        assert g.tensors["q0"].block_size == 64 and g.tensors[f"q{n_t - 1}"].block_size == 64
    assert time.perf_counter() - t0 < 5.0


def valid_file():
    return build([("general.architecture", STR, "llama"), ("llama.block_count", U32, 2)],
                 [("a", [4], 0, bytes(16)), ("b", [8], 0, bytes(32))])


def rejects(write, name, data, match):
    with pytest.raises(VxError, match=match):
        GgufFile(write(name, data))


def test_hostile_headers(write):
    good = valid_file()
    rejects(write, "magic", b"GGUG" + good[4:], "magic")
    for v in (1, 4):
        rejects(write, f"v{v}", good[:4] + struct.pack("<I", v) + good[8:], "version")
    rejects(write, "huge_tensors", good[:8] + struct.pack("<Q", 1 << 60) + good[16:], "tensor count")
    rejects(write, "huge_meta", good[:16] + struct.pack("<Q", 1 << 60) + good[24:], "metadata count")
    body = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 40) + b"k" * 16
    rejects(write, "long_key", body, "longer than the limit")
    key = b"k" * (65537)
    rejects(write, "key_limit", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", len(key)) + key +
            struct.pack("<IB", 0, 1), "longer than the limit")
    rejects(write, "utf8", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28" +
            struct.pack("<IB", 0, 1), "UTF-8")
    arr = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", 9, 4, 1 << 40)
    rejects(write, "array_len", arr, "array length")
    nested = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"a" + struct.pack("<I", 9))
    for _ in range(5):
        nested += struct.pack("<IQ", 9, 1)
    nested += struct.pack("<IQ", 4, 1) + struct.pack("<I", 7)
    rejects(write, "nested", bytes(nested), "nested deeper")
    rejects(write, "type", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"a" + struct.pack("<IB", 13, 0),
            "metadata type")


def test_hostile_tensors(write):
    rejects(write, "align", build([("general.alignment", U32, 24)], [("a", [4], 0, bytes(16))]), "power of two")
    rejects(write, "align_type", build([("general.alignment", STR, "32")], [("a", [4], 0, bytes(16))]), "power of two")
    good = build([], [("a", [16], 0, bytes(64)), ("b", [8], 0, bytes(32))])
    off_b = good.index(b"\x01\x00\x00\x00\x00\x00\x00\x00b") + 9  # b's descriptor after its name
    assert good[off_b:off_b + 4] == struct.pack("<I", 1)
    patched = bytearray(good)
    struct.pack_into("<Q", patched, off_b + 4 + 8 + 4, 32)  # b's offset inside a's payload [0, 64)
    rejects(write, "overlap", bytes(patched), "overlaps")
    struct.pack_into("<Q", patched, off_b + 4 + 8 + 4, 8)
    rejects(write, "misaligned", bytes(patched), "multiple of the alignment")
    struct.pack_into("<Q", patched, off_b + 4 + 8 + 4, 1 << 20)
    rejects(write, "beyond", bytes(patched), "beyond the end")
    struct.pack_into("<I", patched, off_b, 9)
    rejects(write, "dims", bytes(patched), "dimensions")
    rejects(write, "dup", build([], [("a", [4], 0, bytes(16)), ("a", [4], 0, bytes(16))]), "duplicate tensor")
    rejects(write, "dupkey", build([("k", U32, 1), ("k", U32, 2)], []), "duplicate metadata key")
    big = build([], [("a", [1 << 21, 1 << 20], 0, b"")])
    rejects(write, "elements", big, "2\\^40")


def test_truncation_at_every_length_is_an_error(write, tmp_path):
    good = valid_file()
    GgufFile(write("whole", good)).close()
    seen = set()
    for n in range(len(good)):
        p = tmp_path / "cut.gguf"
        p.write_bytes(good[:n])
        with pytest.raises(VxError) as e:
            GgufFile(str(p))
        seen.add(e.value.status)
    assert seen == {8}  # VX_ERR_FORMAT at every length
    with pytest.raises(VxError, match="VX_ERR_IO"):
        GgufFile(str(tmp_path / "does_not_exist.gguf"))


def q2_0_payload(rng, rows, cols, bs):
    """Q2_0 blocks of bs weights with codes 0..2 and random positive f16 scales; returns (bytes, trits, scale bits)."""
    n = rows * cols
    codes = rng.integers(0, 3, n).astype(np.uint8)
    d = (rng.uniform(0.01, 0.1, n // bs).astype(np.float16)).view(np.uint16)
    out = bytearray()
    for b in range(n // bs):
        c = codes[b * bs:(b + 1) * bs].reshape(-1, 4)
        out += struct.pack("<H", d[b]) + bytes((c[:, 0] | c[:, 1] << 2 | c[:, 2] << 4 | c[:, 3] << 6).astype(np.uint8))
    return bytes(out), codes.astype(np.int8) - 1, d


@pytest.mark.parametrize("bs", [64, 128])
def test_q2_0_convert_matches_the_oracle(write, oracle, bs):
    """vx_gguf_convert_q2_0 equals the oracle's Q2_0 decoder (gguf_oracle.c, decode_q2_0 of decoders/q2_0.rs:58-98)
    followed by the planar packer; the scales are the block's f16, once per 64 weights."""
    rng = np.random.default_rng(bs)
    rows, cols = 5, 640
    data, trits, d = q2_0_payload(rng, rows, cols, bs)
    with GgufFile(write("q2", build([], [("w", [cols, rows], 42, data), ("f", [8], 0, bytes(32))]))) as g:
        assert g.tensors["w"].block_size == bs
        planar, scales, r, c = g.convert_q2_0("w")
    want_t, want_s = oracle.q2_0_unpack(np.frombuffer(data, np.uint8), rows, cols, bs)
    assert np.array_equal(want_t.reshape(-1), trits)
    assert (r, c) == (rows, cols)
    assert np.array_equal(planar, oracle.pack_matrix(trits.reshape(rows, cols)).reshape(-1))
    assert np.array_equal(scales, np.asarray(want_s, np.uint16).reshape(-1))
    assert np.array_equal(scales, np.repeat(d, bs // 64))


def test_q2_0_code_3_and_shape_errors(write):
    rng = np.random.default_rng(1)
    data, _, _ = q2_0_payload(rng, 2, 128, 64)
    bad = bytearray(data)
    bad[18 + 2 + 5] |= 3 << 4  # block 1, byte 5, third code: weight 64 + 4 * 5 + 2
    f2 = ("m", [8, 2], 0, bytes(64))
    with GgufFile(write("q2bad", build([], [("w", [128, 2], 42, bytes(bad)), f2, ("f", [8], 0, bytes(32))]))) as g:
        with pytest.raises(VxError, match="weight 86 uses code 3"):
            g.convert_q2_0("w")
        with pytest.raises(VxError, match="not Q2_0"):
            g.convert_q2_0("m")
        with pytest.raises(VxError, match="not a matrix"):
            g.convert_q2_0("f")
