"""numpy front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this module, as the checker or
the timed CPU baseline. The product never imports it. The C sources (velurex_oracle.c) cite the reference file:line
each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libvelurex_oracle.so")

_lib = None


def build() -> None:
    """Compiles the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _declare(L: ctypes.CDLL) -> None:
    vp, sz, u8, f32, u64, uint = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint8, ctypes.c_float,
                                  ctypes.c_uint64, ctypes.c_uint)
    sig = {
        "vxo_pack_5trits": (u8, [vp]),
        "vxo_byte_to_trits": (None, [u8, vp]),
        "vxo_byte_is_valid": (ctypes.c_int, [u8]),
        "vxo_planar_row_bytes": (sz, [sz]),
        "vxo_pack_matrix": (None, [vp, sz, sz, vp]),
        "vxo_unpack_matrix": (None, [vp, sz, sz, vp]),
        "vxo_tile_full_columns": (sz, [sz]),
        "vxo_tile_row_bytes": (sz, [sz]),
        "vxo_column_activation_index": (sz, [sz, sz, sz]),
        "vxo_tile_byte": (u8, [vp, sz, sz]),
        "vxo_untile_row": (None, [vp, sz, vp]),
        "vxo_split_hi_lo": (None, [vp, sz, vp, vp]),
        "vxo_wide_lut_len": (sz, [sz]),
        "vxo_build_compact_wide_lut": (None, [vp, sz, vp]),
        "vxo_decode_u_l": (None, [u8, vp, vp]),
        "vxo_gemv_lut_tilerows": (None, [vp, sz, sz, vp, vp]),
        "vxo_gemv_lut_planar": (None, [vp, sz, sz, vp, vp]),
        "vxo_tile_rows": (None, [vp, sz, sz, vp]),
        "vxo_gemv_bruteforce": (None, [vp, sz, sz, vp, vp]),
        "vxo_epilogue_f32": (None, [vp, sz, f32, f32, vp]),
        "vxo_scale_f32": (None, [vp, sz, f32, vp]),
        "vxo_quantize_i8": (f32, [vp, sz, f32, vp]),
        "vxo_quantize_q8_0": (None, [vp, sz, vp, vp]),
        "vxo_f32_to_f16": (ctypes.c_uint16, [f32]),
        "vxo_f16_to_f32": (f32, [ctypes.c_uint16]),
        "vxo_rms_norm": (None, [vp, vp, sz, f32, vp]),
        "vxo_q2_0_dot_row": (f32, [vp, vp, vp, vp, sz]),
        "vxo_q2_0_gemv": (None, [vp, vp, vp, vp, sz, sz, vp]),
        "vxo_q2_0_lane_sums": (None, [vp, vp, sz, sz, vp]),
        "vxo_gen_trits": (None, [u64, sz, uint, uint, vp]),
        "vxo_gen_i8": (None, [u64, sz, ctypes.c_int, ctypes.c_int, vp]),
        # decode step (decode_oracle.c)
        "vxo_bf16_to_f32": (f32, [ctypes.c_uint16]),
        "vxo_f32_to_bf16": (ctypes.c_uint16, [f32]),
        "vxo_ggml_dot_bf16": (f32, [vp, vp, sz]),
        "vxo_ggml_dot_f16": (f32, [vp, vp, sz]),
        "vxo_vec_mad_f16": (None, [vp, vp, f32, sz]),
        "vxo_vec_scale_f16": (None, [vp, f32, sz]),
        "vxo_expf_batch": (None, [vp, sz, vp]),
        "vxo_rope_cache": (None, [sz, sz, f32, vp]),
        "vxo_rope_neox": (None, [vp, sz, sz, vp, sz]),
        "vxo_rope_normal": (None, [vp, sz, sz, vp, sz]),
        "vxo_ggml_expf": (f32, [f32]),
        "vxo_ggml_expf_batch": (None, [vp, sz, vp]),
        "vxo_swiglu": (None, [vp, vp, sz, vp]),
        "vxo_model_head": (vp, [vp]),
        "vxo_attend_head": (None, [vp, vp, vp, sz, sz, sz, sz, f32, vp]),
        "vxo_projection": (None, [vp, sz, sz, f32, vp, f32, vp]),
        "vxo_projection_shape": (None, [vp, ctypes.c_int, vp, vp]),
        "vxo_model_create": (vp, [vp, u64]),
        "vxo_model_free": (None, [vp]),
        "vxo_model_projection": (vp, [vp, sz, ctypes.c_int, vp]),
        "vxo_model_norm": (vp, [vp, sz, ctypes.c_int]),
        "vxo_model_embedding": (vp, [vp]),
        "vxo_model_rope_table": (vp, [vp]),
        "vxo_model_reset": (None, [vp]),
        "vxo_model_kv_get": (None, [vp, sz, sz, sz, vp, vp]),
        "vxo_model_kv_set": (None, [vp, sz, sz, sz, vp, vp]),
        "vxo_model_forward": (ctypes.c_uint32, [vp, ctypes.c_uint32, sz, vp]),
        "vxo_model_generate": (None, [vp, vp, sz, sz, vp]),
        # GGUF ternary decoders (gguf_oracle.c)
        "vxo_i2s_unpack": (ctypes.c_int, [vp, sz, sz, vp]),
        "vxo_i2s_pack": (ctypes.c_int, [vp, sz, sz, vp]),
        "vxo_tq2_0_unpack": (None, [vp, sz, vp]),
        "vxo_tq1_0_unpack": (None, [vp, sz, vp]),
        "vxo_tq2_0_pack": (None, [vp, sz, ctypes.c_uint16, vp]),
        "vxo_tq1_0_pack": (None, [vp, sz, ctypes.c_uint16, vp]),
        "vxo_q2_0_unpack": (sz, [vp, sz, sz, sz, vp, vp]),
        "vxc_supported": (ctypes.c_int, []),
        "vxc_table_bytes": (sz, [sz]),
        "vxc_tile64": (None, [vp, sz, sz, vp]),
        "vxc_build_tables": (None, [vp, sz, vp]),
        "vxc_gemv_tables": (None, [vp, vp, sz, sz, vp, ctypes.c_int]),
        "vxc_gemv": (None, [vp, vp, sz, sz, vp, ctypes.c_int, vp]),
        "vxc_clock_hz": (ctypes.c_double, []),
        "vxc_gemv_group": (None, [vp, vp, ctypes.c_int, vp, sz, vp, ctypes.c_int, vp]),
        "vxc_fill_valid": (None, [vp, sz, ctypes.c_uint64]),
        "vxc_read_stream": (u64, [vp, sz, ctypes.c_int]),
        "vxc_pin_threads": (ctypes.c_int, [vp, ctypes.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


# ---- encoding ----------------------------------------------------------------------------------------------------

def pack_5trits(t) -> int:
    a = np.ascontiguousarray(t, dtype=np.int8)
    return int(lib().vxo_pack_5trits(_p(a)))


def byte_to_trits(b: int) -> np.ndarray:
    out = np.zeros(5, np.int8)
    lib().vxo_byte_to_trits(b, _p(out))
    return out


def byte_is_valid(b: int) -> bool:
    return bool(lib().vxo_byte_is_valid(b))


def planar_row_bytes(cols: int) -> int:
    return int(lib().vxo_planar_row_bytes(cols))


def pack_matrix(trits: np.ndarray) -> np.ndarray:
    """Planar velurex bytes of a rows x cols trit matrix (rows x planar_row_bytes)."""
    t = np.ascontiguousarray(trits, dtype=np.int8)
    rows, cols = t.shape
    out = np.empty((rows, planar_row_bytes(cols)), np.uint8)
    lib().vxo_pack_matrix(_p(t), rows, cols, _p(out))
    return out


def unpack_matrix(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros((rows, cols), np.int8)
    lib().vxo_unpack_matrix(_p(p), rows, cols, _p(out))
    return out


def tile_full_columns(cols: int) -> int:
    return int(lib().vxo_tile_full_columns(cols))


def tile_row_bytes(cols: int) -> int:
    return int(lib().vxo_tile_row_bytes(cols))


def column_activation_index(cols: int, c: int, p: int) -> int:
    return int(lib().vxo_column_activation_index(cols, c, p))


def tile_row(planar_row: np.ndarray, cols: int) -> np.ndarray:
    r = np.ascontiguousarray(planar_row, dtype=np.uint8)
    return np.array([lib().vxo_tile_byte(_p(r), cols, c) for c in range(tile_row_bytes(cols))], np.uint8)


def tile_rows(planar: np.ndarray, rows: int, cols: int) -> np.ndarray:
    p = np.ascontiguousarray(planar, dtype=np.uint8)
    out = np.empty((rows, tile_row_bytes(cols)), np.uint8)
    lib().vxo_tile_rows(_p(p), rows, cols, _p(out))
    return out


def untile_row(tile_row_bytes_: np.ndarray, cols: int) -> np.ndarray:
    t = np.ascontiguousarray(tile_row_bytes_, dtype=np.uint8)
    out = np.zeros(planar_row_bytes(cols), np.uint8)
    lib().vxo_untile_row(_p(t), cols, _p(out))
    return out


# ---- tables and GEMV ----------------------------------------------------------------------------------------------

def split_hi_lo(acts: np.ndarray):
    a = np.ascontiguousarray(acts, dtype=np.int8)
    hi = np.empty_like(a)
    lo = np.empty_like(a)
    lib().vxo_split_hi_lo(_p(a), a.size, _p(hi), _p(lo))
    return hi, lo


def build_compact_wide_lut(acts: np.ndarray, cols: int) -> np.ndarray:
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty(int(lib().vxo_wide_lut_len(cols)), np.int8)
    lib().vxo_build_compact_wide_lut(_p(a), cols, _p(out))
    return out


def decode_u_l(b: int):
    u = ctypes.c_uint8()
    l = ctypes.c_uint8()
    lib().vxo_decode_u_l(b, ctypes.byref(u), ctypes.byref(l))
    return u.value, l.value


def gemv_lut_planar(planar: np.ndarray, rows: int, cols: int, acts: np.ndarray) -> np.ndarray:
    p = np.ascontiguousarray(planar, dtype=np.uint8)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty(rows, np.int32)
    lib().vxo_gemv_lut_planar(_p(p), rows, cols, _p(a), _p(out))
    return out


def gemv_bruteforce(trits: np.ndarray, acts: np.ndarray) -> np.ndarray:
    t = np.ascontiguousarray(trits, dtype=np.int8)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    rows, cols = t.shape
    out = np.empty(rows, np.int64)
    lib().vxo_gemv_bruteforce(_p(t), rows, cols, _p(a), _p(out))
    return out


def epilogue_f32(acc: np.ndarray, weight_scale: float, act_scale: float) -> np.ndarray:
    a = np.ascontiguousarray(acc, dtype=np.int32)
    out = np.empty(a.size, np.float32)
    lib().vxo_epilogue_f32(_p(a), a.size, weight_scale, act_scale, _p(out))
    return out


def scale_f32(acc: np.ndarray, scale: float) -> np.ndarray:
    a = np.ascontiguousarray(acc, dtype=np.int32)
    out = np.empty(a.size, np.float32)
    lib().vxo_scale_f32(_p(a), a.size, scale, _p(out))
    return out


# ---- quantizers, norms ---------------------------------------------------------------------------------------------

def quantize_i8(x: np.ndarray, levels: float = 127.0):
    v = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(v.size, np.int8)
    s = lib().vxo_quantize_i8(_p(v), v.size, levels, _p(q))
    return q, float(np.float32(s))


def quantize_q8_0(x: np.ndarray):
    v = np.ascontiguousarray(x, dtype=np.float32)
    qs = np.empty(v.size, np.int8)
    d = np.empty(v.size // 32, np.float32)
    lib().vxo_quantize_q8_0(_p(v), v.size, _p(qs), _p(d))
    return qs, d


def f32_to_f16_bits(x: float) -> int:
    return int(lib().vxo_f32_to_f16(x))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().vxo_f16_to_f32(h))


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    xv = np.ascontiguousarray(x, dtype=np.float32)
    wv = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(xv)
    lib().vxo_rms_norm(_p(xv), _p(wv), xv.size, eps, _p(out))
    return out


# ---- Q2_0 -------------------------------------------------------------------------------------------------------

def q2_0_gemv(packed: np.ndarray, w_scales: np.ndarray, acts: np.ndarray, a_scales: np.ndarray, rows: int,
              cols: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    ws = np.ascontiguousarray(w_scales, dtype=np.float32)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    as_ = np.ascontiguousarray(a_scales, dtype=np.float32)
    out = np.empty(rows, np.float32)
    lib().vxo_q2_0_gemv(_p(p), _p(ws), _p(a), _p(as_), rows, cols, _p(out))
    return out


def q2_0_lane_sums(packed: np.ndarray, acts: np.ndarray, rows: int, cols: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty((rows, cols // 32, 8), np.int32)
    lib().vxo_q2_0_lane_sums(_p(p), _p(a), rows, cols, _p(out))
    return out


# ---- generators ----------------------------------------------------------------------------------------------------

def gen_trits(seed: int, shape, p_minus: int = 35, p_zero: int = 30) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.int8)
    lib().vxo_gen_trits(seed, n, p_minus, p_zero, _p(out))
    return out.reshape(shape)


def gen_i8(seed: int, n: int, lo: int = -127, hi: int = 127) -> np.ndarray:
    out = np.empty(n, np.int8)
    lib().vxo_gen_i8(seed, n, lo, hi, _p(out))
    return out


# ---- decode step (decode_oracle.c) ----------------------------------------------------------------------------------

ACT_RELU2, ACT_SILU = 0, 1
ROPE_NEOX, ROPE_NORMAL = 0, 1


class ModelConfig(ctypes.Structure):
    """vxo_model_config: the decoder shape and its architecture switches (all zero: the BitNet of BASELINE.json
    configs[3], bitnet_2b(); falcon3() sets SiLU, Normal RoPE, no sub-norms, an f16 embedding and an untied f16 head)."""
    _fields_ = [("n_layers", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
                ("n_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32), ("ffn", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("max_ctx", ctypes.c_uint32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("act", ctypes.c_uint32), ("rope_mode", ctypes.c_uint32),
                ("no_sub_norm", ctypes.c_uint32), ("emb_f16", ctypes.c_uint32), ("untied", ctypes.c_uint32)]

    @property
    def is_falcon3(self) -> bool:
        return self.act == ACT_SILU


def bitnet_2b(max_ctx: int = 4096) -> ModelConfig:
    """ModelConfig::bitnet_2b_default (quintrit-runtime/src/config.rs:155-177)."""
    return ModelConfig(30, 2560, 20, 5, 128, 6912, 128256, max_ctx, 1e-5, 500000.0)


def falcon3(n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx, rms_eps=1e-5,
            rope_theta=100000.0) -> ModelConfig:
    """A Falcon3-architecture config (ModelConfig::falcon3_*_default, config.rs:179-227): SiLU / SwiGLU, Normal RoPE,
    no sub-norms, f16 embedding and an untied f16 head."""
    return ModelConfig(n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx, rms_eps, rope_theta,
                       ACT_SILU, ROPE_NORMAL, 1, 1, 1)


def falcon3_10b(max_ctx: int = 4096, n_layers: int = 40) -> ModelConfig:
    """BASELINE.json configs[1]'s Falcon3-10B shapes (40 layers, hidden 3072, 12 / 4 heads of 256, FFN 23040) with the
    Falcon3 vocabulary (131072) and the other constants of falcon3_7b_default (config.rs:205-227)."""
    return falcon3(n_layers, 3072, 12, 4, 256, 23040, 131072, max_ctx)


PROJ_NAMES = ("q", "k", "v", "o", "gate", "up", "down")


class Model:
    """The oracle's decoder with weights generated from a seed (vxo_model_*)."""

    def __init__(self, cfg: ModelConfig, seed: int):
        self.cfg = cfg
        self._h = lib().vxo_model_create(ctypes.byref(cfg), seed)
        if not self._h:
            raise ValueError("unsupported model shape")

    def close(self):
        if self._h:
            lib().vxo_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def projection_shape(self, kind: int):
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        lib().vxo_projection_shape(ctypes.byref(self.cfg), kind, ctypes.byref(r), ctypes.byref(c))
        return r.value, c.value

    def projection(self, layer: int, kind: int):
        """(planar bytes, weight scale) of projection `kind` of `layer` (a copy)."""
        ws = ctypes.c_float()
        p = lib().vxo_model_projection(self._h, layer, kind, ctypes.byref(ws))
        rows, cols = self.projection_shape(kind)
        n = rows * planar_row_bytes(cols)
        return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(p)).copy(), float(ws.value)

    def norm(self, layer: int, kind: int):
        """RMSNorm weights (a copy), or None for a sub-norm of a model without them."""
        c = self.cfg
        n = c.ffn if kind == 3 else (c.n_heads * c.head_dim if kind == 1 else c.hidden)
        if layer == c.n_layers:
            n = c.hidden
        p = lib().vxo_model_norm(self._h, layer, kind)
        if not p:
            return None
        return np.ctypeslib.as_array((ctypes.c_float * n).from_address(p)).copy()

    def embedding(self) -> np.ndarray:
        """bf16 or f16 bits (cfg.emb_f16), vocab x hidden, a view into the model."""
        n = self.cfg.vocab * self.cfg.hidden
        p = lib().vxo_model_embedding(self._h)
        return np.ctypeslib.as_array((ctypes.c_uint16 * n).from_address(p)).reshape(self.cfg.vocab, self.cfg.hidden)

    def head(self) -> np.ndarray:
        """The head (the embedding when tied), same type, a view into the model."""
        n = self.cfg.vocab * self.cfg.hidden
        p = lib().vxo_model_head(self._h)
        return np.ctypeslib.as_array((ctypes.c_uint16 * n).from_address(p)).reshape(self.cfg.vocab, self.cfg.hidden)

    def rope_table(self) -> np.ndarray:
        n = self.cfg.max_ctx * self.cfg.head_dim
        p = lib().vxo_model_rope_table(self._h)
        return np.ctypeslib.as_array((ctypes.c_float * n).from_address(p)).reshape(self.cfg.max_ctx, self.cfg.head_dim)

    def reset(self):
        lib().vxo_model_reset(self._h)

    def kv(self, layer: int, pos: int, kv_head: int):
        """The cached f16 key and value bits (uint16 arrays of head_dim) of (layer, pos, kv_head)."""
        k = np.empty(self.cfg.head_dim, np.uint16)
        v = np.empty(self.cfg.head_dim, np.uint16)
        lib().vxo_model_kv_get(self._h, layer, pos, kv_head, _p(k), _p(v))
        return k, v

    def set_kv(self, layer: int, pos: int, kv_head: int, k, v) -> None:
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        lib().vxo_model_kv_set(self._h, layer, pos, kv_head, _p(k), _p(v))

    def forward(self, token: int, pos: int):
        logits = np.empty(self.cfg.vocab, np.float32)
        nxt = lib().vxo_model_forward(self._h, token, pos, _p(logits))
        return int(nxt), logits

    def generate(self, prompt, n_new: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n_new, np.uint32)
        lib().vxo_model_generate(self._h, _p(p), p.size, n_new, _p(out))
        return out


def f32_to_bf16(x: float) -> int:
    return int(lib().vxo_f32_to_bf16(x))


def bf16_to_f32(h: int) -> float:
    return float(lib().vxo_bf16_to_f32(h))


def ggml_dot_bf16(x: np.ndarray, y: np.ndarray) -> float:
    a, b = np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(y, np.uint16)
    return float(np.float32(lib().vxo_ggml_dot_bf16(_p(a), _p(b), a.size)))


def ggml_dot_f16(x: np.ndarray, y: np.ndarray) -> float:
    a, b = np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(y, np.uint16)
    return float(np.float32(lib().vxo_ggml_dot_f16(_p(a), _p(b), a.size)))


def vec_mad_f16(y: np.ndarray, x: np.ndarray, v: float) -> np.ndarray:
    out = np.ascontiguousarray(y, np.uint16).copy()
    xx = np.ascontiguousarray(x, np.uint16)
    lib().vxo_vec_mad_f16(_p(out), _p(xx), v, out.size)
    return out


def vec_scale_f16(y: np.ndarray, v: float) -> np.ndarray:
    out = np.ascontiguousarray(y, np.uint16).copy()
    lib().vxo_vec_scale_f16(_p(out), v, out.size)
    return out


def expf(x: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    lib().vxo_expf_batch(_p(a), a.size, _p(out))
    return out


def rope_cache(pos: int, n_dims: int, base: float) -> np.ndarray:
    out = np.empty(n_dims, np.float32)
    lib().vxo_rope_cache(pos, n_dims, base, _p(out))
    return out


def rope_neox(x: np.ndarray, heads: int, head_dim: int, cache: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(x, np.float32).copy()
    c = np.ascontiguousarray(cache, np.float32)
    lib().vxo_rope_neox(_p(out), heads, head_dim, _p(c), c.size)
    return out


def rope_normal(x: np.ndarray, heads: int, head_dim: int, cache: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(x, np.float32).copy()
    c = np.ascontiguousarray(cache, np.float32)
    lib().vxo_rope_normal(_p(out), heads, head_dim, _p(c), c.size)
    return out


def ggml_expf(x: float) -> float:
    return float(np.float32(lib().vxo_ggml_expf(float(x))))


def ggml_expf_array(x: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    lib().vxo_ggml_expf_batch(_p(a), a.size, _p(out))
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g, u = np.ascontiguousarray(gate, np.float32), np.ascontiguousarray(up, np.float32)
    out = np.empty_like(g)
    lib().vxo_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def attend_head(q_f16, k_f16, v_f16, seq_len: int, max_ctx: int, scale: float) -> np.ndarray:
    """One head over k/v rows [0, seq_len) (arrays [positions][head_dim] of f16 bits)."""
    q = np.ascontiguousarray(q_f16, np.uint16)
    k = np.ascontiguousarray(k_f16, np.uint16)
    v = np.ascontiguousarray(v_f16, np.uint16)
    out = np.empty(q.size, np.float32)
    lib().vxo_attend_head(_p(q), _p(k), _p(v), q.size, q.size, seq_len, max_ctx, scale, _p(out))
    return out


# ---- the AVX-512 transcription of the reference's production CPU GEMV (cpu_avx512.c; the CPU baseline) ----------

def cpu_avx512_supported() -> bool:
    return bool(lib().vxc_supported())


def tile64(planar: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Planar rows -> the reference's 64-row tiled layout (transform_weights_lut_64); rows a multiple of 64."""
    p = np.ascontiguousarray(planar, dtype=np.uint8)
    out = np.empty(rows * tile_row_bytes(cols), np.uint8)
    lib().vxc_tile64(_p(p), rows, cols, _p(out))
    return out


def gemv_avx512(tiles64_: np.ndarray, acts: np.ndarray, rows: int, cols: int, threads: int = 1) -> np.ndarray:
    """float(sum_k t[r][k] acts[k]) by the AVX-512 kernel (raises when the host lacks AVX-512 VBMI)."""
    if not cpu_avx512_supported():
        raise RuntimeError("this host has no AVX-512 F/BW/VBMI")
    t = np.ascontiguousarray(tiles64_, dtype=np.uint8)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty(rows, np.float32)
    scratch = np.empty(int(lib().vxc_table_bytes(cols)), np.int8)
    lib().vxc_gemv(_p(t), _p(a), rows, cols, _p(out), threads, _p(scratch))
    return out


def gemv_group_avx512(tiles: list, rows: list, acts: np.ndarray, cols: int, threads: int = 1) -> list:
    """One projection group (matrices sharing the input acts) by the AVX-512 kernel: one table build, the group's
    blocks split over `threads` threads; returns one float32 vector per matrix."""
    if not cpu_avx512_supported():
        raise RuntimeError("this host has no AVX-512 F/BW/VBMI")
    ts = [np.ascontiguousarray(t, dtype=np.uint8) for t in tiles]
    a = np.ascontiguousarray(acts, dtype=np.int8)
    outs = [np.empty(r, np.float32) for r in rows]
    n = len(ts)
    tp = (ctypes.c_void_p * n)(*[t.ctypes.data for t in ts])
    op = (ctypes.c_void_p * n)(*[o.ctypes.data for o in outs])
    rp = (ctypes.c_size_t * n)(*rows)
    scratch = np.empty(int(lib().vxc_table_bytes(cols)), np.int8)
    lib().vxc_gemv_group(ctypes.cast(tp, ctypes.c_void_p), ctypes.cast(rp, ctypes.c_void_p), n, _p(a), cols,
                         ctypes.cast(op, ctypes.c_void_p), threads, _p(scratch))
    return outs


# ---- GGUF ternary decoders (gguf_oracle.c) -------------------------------------------------------------------------

GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q8_0, GGML_TYPE_BF16 = 0, 1, 8, 30
GGML_TYPE_TQ1_0, GGML_TYPE_TQ2_0, GGML_TYPE_I2_S, GGML_TYPE_Q2_0 = 34, 35, 36, 42


def i2s_unpack(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, np.uint8)
    out = np.empty(rows * cols, np.int8)
    if lib().vxo_i2s_unpack(_p(p), rows, cols, _p(out)) != 0:
        raise ValueError("I2_S cols must be a multiple of 128")
    return out.reshape(rows, cols)


def i2s_pack(trits: np.ndarray) -> np.ndarray:
    t = np.ascontiguousarray(trits, np.int8)
    rows, cols = t.shape
    out = np.empty(rows * cols // 4, np.uint8)
    if lib().vxo_i2s_pack(_p(t), rows, cols, _p(out)) != 0:
        raise ValueError("I2_S cols must be a multiple of 128")
    return out


def tq_unpack(ty: int, data: np.ndarray, n: int) -> np.ndarray:
    """The n trits of TQ1_0 (34) or TQ2_0 (35) blocks."""
    d = np.ascontiguousarray(data, np.uint8)
    out = np.empty(n, np.int8)
    (lib().vxo_tq1_0_unpack if ty == GGML_TYPE_TQ1_0 else lib().vxo_tq2_0_unpack)(_p(d), n // 256, _p(out))
    return out


def tq_pack(ty: int, trits: np.ndarray, d_bits: int = 0x3800) -> np.ndarray:
    t = np.ascontiguousarray(trits, np.int8).reshape(-1)
    nb = t.size // 256
    out = np.empty(nb * (54 if ty == GGML_TYPE_TQ1_0 else 66), np.uint8)
    (lib().vxo_tq1_0_pack if ty == GGML_TYPE_TQ1_0 else lib().vxo_tq2_0_pack)(_p(t), nb, d_bits, _p(out))
    return out


def q2_0_unpack(data: np.ndarray, rows: int, cols: int, block_size: int = 64):
    """(trits rows x cols, f16 scale bits per 64 weights); raises on a code 3 weight."""
    d = np.ascontiguousarray(data, np.uint8)
    trits = np.empty(rows * cols, np.int8)
    scales = np.empty(rows * cols // 64, np.uint16)
    bad = lib().vxo_q2_0_unpack(_p(d), rows, cols, block_size, _p(trits), _p(scales))
    if bad:
        raise ValueError(f"Q2_0 weight {bad - 1} uses code 3")
    return trits.reshape(rows, cols), scales
