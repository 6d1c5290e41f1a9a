"""The C ABI (include/velurex_hip.h) on the CPU: the library loads, exports every declared symbol, keeps the reference's
status codes, computes the device layout on the host and rejects bad arguments before any GPU work."""
import ctypes
import os
import re

import numpy as np
import pytest

from quintrit_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "velurex_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_status_codes_match_the_reference():
    # quintrit-c/include/quintrit.h:73-88
    want = {"VX_OK": 0, "VX_ERR_NULL_POINTER": 1, "VX_ERR_INVALID_ARGUMENT": 2, "VX_ERR_INVALID_SHAPE": 3,
            "VX_ERR_BUFFER_TOO_SMALL": 4, "VX_ERR_INVALID_VALUE": 5, "VX_ERR_UNSUPPORTED": 6, "VX_ERR_IO": 7,
            "VX_ERR_FORMAT": 8, "VX_ERR_NOT_FOUND": 9, "VX_ERR_MODEL": 10, "VX_ERR_CONTEXT_OVERFLOW": 11,
            "VX_ERR_BUSY": 12, "VX_ERR_INTERNAL": 13, "VX_ERR_INVALID_HANDLE": 14, "VX_ERR_DEVICE": 15}
    text = open(HEADER).read()
    for name, value in want.items():
        m = re.search(rf"#define {name}\s+(\d+)", text)
        assert m and int(m.group(1)) == value, name
        assert _lib.STATUS_NAMES[value] == name
    L = _lib.lib()
    assert L.vx_status_string(0) == b"ok"
    assert L.vx_status_string(999) == b"unknown status"
    assert L.vx_abi_version() == 2 and L.vx_version() == b"0.2.0"


def test_layout_matches_the_oracle(oracle):
    for rows, cols in [(1, 1), (64, 160), (65, 161), (3072, 3072), (23040, 3072), (3072, 23040), (7, 4096), (1100, 160)]:
        lay = _lib.layout(rows, cols)
        assert lay["tile_rows"] == 64
        assert lay["padded_rows"] == -(-rows // 64) * 64
        assert lay["planar_row_bytes"] == oracle.planar_row_bytes(cols)
        assert lay["tile_row_bytes"] == oracle.tile_row_bytes(cols)
        assert lay["device_row_bytes"] == -(-oracle.tile_row_bytes(cols) // 16) * 16
        assert lay["device_bytes"] == lay["padded_rows"] * lay["device_row_bytes"]


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 161), (64, 160), (70, 3072), (130, 4096), (5, 23040), (1100, 160),
                                       (2049, 321)])
def test_device_layout_pack_places_every_byte(oracle, rows, cols):
    # The device layout (velurex_hip.h, vx_layout): tile row bytes (the oracle's tile_byte, pack.rs:240-256) in 16-byte
    # chunks; chunk q of tile t sits at KiB g*16*n_chunks + q*T + t%16 (g = t//16, T = tiles of group g); padding is
    # byte 125 (five zero trits).
    rng = np.random.default_rng(rows * 7 + cols)
    trits = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    planar = oracle.pack_matrix(trits)
    dev = _lib.device_layout_pack(planar, rows, cols)
    lay = _lib.layout(rows, cols)
    dbr, tbr = lay["device_row_bytes"], lay["tile_row_bytes"]
    want = np.full((lay["padded_rows"], dbr), 125, np.uint8)
    for r in range(rows):
        want[r, :tbr] = oracle.tile_row(planar[r], cols)
    n_tiles, n_chunks = lay["padded_rows"] // 64, dbr // 16
    tiles = want.reshape(n_tiles, 64, n_chunks, 16).transpose(0, 2, 1, 3)  # [tile][chunk][row][16]
    parts = []
    for g0 in range(0, n_tiles, 16):
        grp = tiles[g0:g0 + 16]                                               # [T][chunk][row][16]
        parts.append(grp.transpose(1, 0, 2, 3).reshape(-1))                  # chunk-major, then tile
    assert lay["tile_group"] == 16
    assert np.array_equal(dev, np.concatenate(parts))


def test_invalid_bytes_are_rejected(oracle):
    planar = oracle.pack_matrix(np.zeros((2, 160), np.int8))
    for bad in (27, 251, 255):
        p = planar.copy()
        p[1, 5] = bad
        with pytest.raises(_lib.VxError) as e:
            _lib.device_layout_pack(p, 2, 160)
        assert e.value.status == 5  # VX_ERR_INVALID_VALUE
        assert "byte 37" in str(e.value)


def test_argument_errors_without_gpu():
    L = _lib.lib()
    vp = ctypes.c_void_p
    buf = (ctypes.c_uint8 * 64)()
    h = vp()
    assert L.vx_matrix_create(None, 0, 1, 1, 1.0, ctypes.byref(h)) == 1          # NULL planar
    assert L.vx_matrix_create(buf, 64, 0, 1, 1.0, ctypes.byref(h)) == 3          # rows = 0
    assert L.vx_matrix_create(buf, 64, 1, 131073, 1.0, ctypes.byref(h)) == 3     # cols too large
    assert L.vx_matrix_create(buf, 16, 1, 160, 1.0, ctypes.byref(h)) == 4        # planar too short
    assert b"needs 32" in L.vx_last_error_message()
    assert L.vx_last_error_code() == 4
    assert L.vx_matrix_free(None) == 0
    assert L.vx_gemv_i32_dev(None, buf, 1, buf, 1, None) == 14                   # NULL handle
    lay = _lib._Layout()
    lay.struct_size = 3
    assert L.vx_layout(1, 1, ctypes.byref(lay)) == 2                              # wrong struct_size
    with pytest.raises(_lib.VxError):
        _lib.staged_bytes(0)
    assert _lib.staged_bytes(3072) == 64 + 624 * 8
    # plans: argument checks happen before any device work
    jobs = (_lib.GemvJob * 1)()
    jobs[0].struct_size = ctypes.sizeof(_lib.GemvJob)
    assert L.vx_plan_create(jobs, 0, ctypes.byref(h)) == 2                       # no jobs
    assert L.vx_plan_create(None, 1, ctypes.byref(h)) == 1                       # NULL jobs
    assert L.vx_plan_run(None, None) == 14                                        # NULL plan
    assert L.vx_plan_free(None) == 0
    n = ctypes.c_size_t()
    assert L.vx_gemm_workspace_bytes(None, 8, ctypes.byref(n)) == 14               # NULL handle
    assert L.vx_gemm_i32_dev(None, buf, 8, 64, buf, 64, buf, 64, None) == 14
    # Q2_0: shape rules before any device work (cols a multiple of 64, at most 12288)
    assert L.vx_q2_matrix_create(buf, 64, buf, 64, 1, 100, ctypes.byref(h)) == 3
    assert L.vx_q2_matrix_create(buf, 64, buf, 64, 1, 12352, ctypes.byref(h)) == 3
    assert L.vx_q2_matrix_create(buf, 16, buf, 64, 1, 64, ctypes.byref(h)) == 4   # planar too short
    assert L.vx_q2_gemv_f32_dev(None, buf, 64, buf, 2, buf, 1, None) == 14
    # compact activation tables: 2 x 64 bytes per tile-row byte (avx512.rs:935-938), checks before any device work
    assert _lib.compact_lut_bytes(3072) == 2 * 64 * 616
    assert _lib.compact_lut_bytes(161) == 2 * 64 * 34
    assert L.vx_compact_lut_bytes(3072, None) == 1                               # NULL out
    assert L.vx_compact_lut_dev(None, 8, 8, buf, 64, None) == 1                   # NULL activations
    assert L.vx_compact_lut_dev(buf, 4, 8, buf, 64 * 4, None) == 4                # activations too short
    assert L.vx_compact_lut_dev(buf, 160, 160, buf, 2 * 64 * 32 - 1, None) == 4   # table buffer too short
    assert L.vx_gemv_lut_i32_dev(None, buf, 64, buf, 1, None) == 14               # NULL handle
    assert L.vx_lut_plan_create(None, 1, ctypes.byref(h)) == 1                    # NULL jobs


def test_decoder_config_errors_before_device():
    """vx_decoder_create checks its configuration before touching a device (so these run without a GPU)."""
    import ctypes
    from quintrit_amd import _lib
    from quintrit_amd.decoder import DecoderConfig
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.vx_decoder_create(None, ctypes.byref(h)) == 1  # NULL config
    c = DecoderConfig.bitnet_2b()._c()
    c.struct_size = 4
    assert L.vx_decoder_create(ctypes.byref(c), ctypes.byref(h)) == 2
    for field, value, status in (("head_dim", 96, 6), ("max_ctx", 8193, 6), ("n_kv_heads", 3, 2), ("hidden", 100, 6),
                                 ("ffn", 9000, 6), ("vocab", 0, 2), ("n_layers", 0, 2)):
        c = DecoderConfig.bitnet_2b()._c()
        setattr(c, field, value)
        assert L.vx_decoder_create(ctypes.byref(c), ctypes.byref(h)) == status, field
        assert field.split("_")[0] in L.vx_last_error_message().decode() or status == 2
    assert L.vx_decoder_free(None) == 0
    assert L.vx_decoder_step(None, 0, 0, None, 0, None) == 14
