"""GGUF model files and their ternary tensors over vx_gguf_* (include/velurex_hip.h).

Mirrors the reference's reader and transcoder (quintrit-format/src/gguf.rs: GgufFile with its metadata, tensors,
get_tensor_data, get_tensor_scale, typed accessors and architecture helpers; transcoder.rs: transcode_to_planar and
load_and_transcode_gguf_tensor). Parsing and the host conversion run in libvelurex_hip.so on the CPU; upload_matrix
converts in HBM. Errors surface as VxError (VX_ERR_IO for a file that cannot be opened, VX_ERR_FORMAT for a malformed or
hostile file).
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass

import numpy as np

from ._lib import VxError, check, lib

GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q8_0, GGML_TYPE_BF16 = 0, 1, 8, 30
GGML_TYPE_TQ1_0, GGML_TYPE_TQ2_0, GGML_TYPE_I2_S, GGML_TYPE_Q2_0 = 34, 35, 36, 42
TERNARY_TYPES = (GGML_TYPE_I2_S, GGML_TYPE_TQ1_0, GGML_TYPE_TQ2_0)


class _Info(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("version", ctypes.c_uint32), ("tensor_count", ctypes.c_uint64),
                ("metadata_count", ctypes.c_uint64), ("data_offset", ctypes.c_uint64)]


class _TensorInfo(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("ggml_type", ctypes.c_int32), ("n_dims", ctypes.c_uint32),
                ("is_ternary", ctypes.c_int32), ("shape", ctypes.c_uint64 * 8), ("num_elements", ctypes.c_uint64),
                ("offset", ctypes.c_uint64), ("data_bytes", ctypes.c_uint64), ("name", ctypes.c_char_p),
                ("type_name", ctypes.c_char_p), ("block_size", ctypes.c_uint32)]


@dataclass(frozen=True)
class GgufTensorInfo:
    """gguf.rs GgufTensorInfo: shape as stored (shape[0] innermost), type, offset in the data section, byte length (0
    when the layout of the type is not known) and the Q2_0 block size (None for other types)."""

    name: str
    shape: tuple
    tensor_type: int
    offset: int
    byte_len: int
    block_size: int | None
    type_name: str

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


def _typed(vtype: int, array_type, value):
    """JSON prints integral floats without a point: floats (types 6, 12) become Python floats again, bools (7) bools;
    nested arrays carry no element type, so only their first level is typed."""
    if vtype in (6, 12):
        return float(value)
    if vtype == 7:
        return bool(value)
    if vtype == 9 and array_type is not None:
        return [_typed(array_type, None, v) for v in value]
    return value


class GgufFile:
    """An open, memory-mapped GGUF v2/v3 file (GgufFile::open)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().vx_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        info = _Info()
        info.struct_size = ctypes.sizeof(_Info)
        check(lib().vx_gguf_info(self._h, ctypes.byref(info)))
        self.version = info.version
        self.data_start = info.data_offset
        n = ctypes.c_size_t()
        st = lib().vx_gguf_metadata_json(self._h, None, 0, ctypes.byref(n))
        if st not in (0, 4):
            check(st)
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().vx_gguf_metadata_json(self._h, buf, n.value + 1, ctypes.byref(n)))
        raw = json.loads(buf.value.decode("utf-8"))
        self.metadata_types = {k: (v["type"], v.get("array_type")) for k, v in raw.items()}
        self.metadata = {k: _typed(v["type"], v.get("array_type"), v["value"]) for k, v in raw.items()}
        self.tensors = {}
        self._order = []
        for i in range(info.tensor_count):
            t = _TensorInfo()
            t.struct_size = ctypes.sizeof(_TensorInfo)
            check(lib().vx_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            name = t.name.decode("utf-8")
            self.tensors[name] = GgufTensorInfo(name, tuple(t.shape[:t.n_dims]), t.ggml_type, t.offset, t.data_bytes,
                                                t.block_size or None, t.type_name.decode())
            self._order.append(name)
        self._read = set()

    def close(self) -> None:
        if self._h:
            check(lib().vx_gguf_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def get_tensor_data(self, name: str):
        """The raw payload as a read-only uint8 view into the mapping, or None for a missing tensor or a type whose
        layout is not known (gguf.rs:318-340). Valid while the file is open."""
        if name not in self.tensors:
            return None
        self._read.add(name)
        p, n = ctypes.POINTER(ctypes.c_uint8)(), ctypes.c_size_t()
        st = lib().vx_gguf_tensor_data(self._h, name.encode(), ctypes.byref(p), ctypes.byref(n))
        if st != 0:
            return None
        arr = np.ctypeslib.as_array(p, shape=(n.value,)) if n.value else np.empty(0, np.uint8)
        arr.flags.writeable = False
        return arr

    def get_tensor_scale(self, name: str) -> float:
        """The per-tensor weight scale (I2_S trailing f32, TQ common block scale, else 1.0); VxError for TQ tensors
        whose blocks differ."""
        s = ctypes.c_float()
        check(lib().vx_gguf_tensor_scale(self._h, name.encode(), ctypes.byref(s)))
        return float(s.value)

    def get_tensor_f32(self, name: str):
        t = self.tensors.get(name)
        if t is None or t.tensor_type != GGML_TYPE_F32:
            return None
        return self.get_tensor_data(name).view(np.float32).copy()

    def get_tensor_f16(self, name: str):
        """Raw f16 bits (uint16)."""
        t = self.tensors.get(name)
        if t is None or t.tensor_type != GGML_TYPE_F16:
            return None
        return self.get_tensor_data(name).view(np.uint16)

    def unread_tensors(self) -> list:
        return sorted(n for n in self._order if n not in self._read)

    # architecture helpers (gguf.rs:384-452)
    def architecture(self):
        v = self.metadata.get("general.architecture")
        return v if isinstance(v, str) else None

    def _arch_key(self, suffix: str):
        a = self.architecture()
        return None if a is None else self.metadata.get(f"{a}.{suffix}")

    def _arch_uint(self, suffix: str):
        v = self._arch_key(suffix)
        return v if isinstance(v, int) and not isinstance(v, bool) and v >= 0 else None

    def context_length(self):
        return self._arch_uint("context_length")

    def embedding_length(self):
        return self._arch_uint("embedding_length")

    def block_count(self):
        return self._arch_uint("block_count")

    def feed_forward_length(self):
        return self._arch_uint("feed_forward_length")

    def head_count(self):
        return self._arch_uint("attention.head_count")

    def head_count_kv(self):
        return self._arch_uint("attention.head_count_kv")

    def vocab_size(self):
        return self._arch_uint("vocab_size")

    def rms_norm_eps(self):
        v = self._arch_key("attention.layer_norm_rms_epsilon")
        return float(v) if isinstance(v, float) else None

    def rope_freq_base(self):
        v = self._arch_key("rope.freq_base")
        return float(v) if isinstance(v, float) else None

    # transcoding (transcoder.rs)
    def convert_planar(self, name: str):
        """(planar velurex bytes, rows, cols, weight scale) of a ternary 2-D tensor, converted on the host."""
        t = self.tensors[name]
        if len(t.shape) != 2:
            raise VxError(3, f"tensor '{name}' is not a matrix")
        cols, rows = t.shape
        out = np.empty(rows * ((cols + 159) // 160) * 32, np.uint8)
        r, c, s = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_float()
        check(lib().vx_gguf_convert_planar(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size,
                                           ctypes.byref(r), ctypes.byref(c), ctypes.byref(s)))
        self._read.add(name)
        return out, r.value, c.value, float(s.value)

    def convert_q2_0(self, name: str):
        """(planar velurex bytes, f16 scale bits (uint16, one per 64 weights of a row), rows, cols) of a Q2_0 matrix
        (decode_q2_0_packed); VxError for a code 3."""
        t = self.tensors[name]
        if len(t.shape) != 2:
            raise VxError(3, f"tensor '{name}' is not a matrix")
        cols, rows = t.shape
        planar = np.empty(rows * ((cols + 159) // 160) * 32, np.uint8)
        scales = np.empty(max(rows * cols // 64, 1), np.uint16)
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().vx_gguf_convert_q2_0(self._h, name.encode(), planar.ctypes.data_as(ctypes.c_void_p), planar.size,
                                         scales.ctypes.data_as(ctypes.c_void_p), scales.size, ctypes.byref(r),
                                         ctypes.byref(c)))
        self._read.add(name)
        return planar, scales[:rows * cols // 64], r.value, c.value

    def upload_q2_matrix(self, name: str):
        """A Q2_0 GEMV matrix (Q2Matrix) from a Q2_0 tensor."""
        from ._lib import Q2Matrix
        h = ctypes.c_void_p()
        check(lib().vx_gguf_upload_q2_matrix(self._h, name.encode(), ctypes.byref(h)))
        self._read.add(name)
        cols, rows = self.tensors[name].shape
        return Q2Matrix._from_handle(h, rows, cols)

    def upload_matrix(self, name: str):
        """A GEMV matrix (VelurexHipLayer) from a ternary tensor, converted on the GPU."""
        from .layer import VelurexHipLayer
        h = ctypes.c_void_p()
        check(lib().vx_gguf_upload_matrix(self._h, name.encode(), ctypes.byref(h)))
        self._read.add(name)
        return VelurexHipLayer._from_handle(h)


def ggml_to_planar(ggml_type: int, data, rows: int, cols: int) -> np.ndarray:
    """transcode_to_planar (transcoder.rs:154-205) for a raw payload: the planar velurex bytes of rows x cols weights."""
    d = np.ascontiguousarray(data, np.uint8).reshape(-1)
    out = np.empty(rows * ((cols + 159) // 160) * 32, np.uint8)
    check(lib().vx_ggml_to_planar(ggml_type, d.ctypes.data_as(ctypes.c_void_p), d.size, rows, cols,
                                  out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out
