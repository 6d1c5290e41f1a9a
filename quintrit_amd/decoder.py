"""Greedy decoding of a ternary (BitNet-b1.58 or Falcon3 family) model on the GPU: the token loop of vx_decoder_* in
include/velurex_hip.h.

Mirrors the reference's runtime surface for this path: ModelConfig (quintrit-runtime/src/config.rs:155-227),
QuintritModel::forward_token (model.rs:282-377: one token at one position, logits out) and the greedy generation loop
(engine.rs:590-686 with Sampler::sample greedy, sampler.rs:73-83). Weights are handed over as the reference holds them:
planar velurex bytes with a per-tensor scale per projection, f32 RMSNorm weights, a bf16 or f16 embedding that is also
the head unless the model has its own (Falcon3's lm_head). Everything runs in libvelurex_hip.so; without it (or
without a gfx950 GPU) construction raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib

PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN = range(7)
NORM_ATTN, NORM_ATTN_SUB, NORM_FFN, NORM_FFN_SUB = range(4)
ACT_RELU2, ACT_SILU = 0, 1
ROPE_NEOX, ROPE_NORMAL = 0, 1


class _Config(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("n_layers", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("n_heads", ctypes.c_uint32), ("n_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("ffn", ctypes.c_uint32), ("vocab", ctypes.c_uint32), ("max_ctx", ctypes.c_uint32),
                ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("act", ctypes.c_uint32),
                ("rope_mode", ctypes.c_uint32), ("no_sub_norm", ctypes.c_uint32), ("emb_f16", ctypes.c_uint32),
                ("untied", ctypes.c_uint32)]


@dataclass(frozen=True)
class DecoderConfig:
    """The model shape (ModelConfig): layers, widths, heads, vocabulary, context, the RMSNorm/RoPE constants and the
    architecture switches (all 0: BitNet with a tied bf16 head; falcon3(): SiLU, Normal RoPE, no sub-norms, f16
    embedding and an untied f16 head)."""

    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_ctx: int
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    act: int = ACT_RELU2
    rope_mode: int = ROPE_NEOX
    no_sub_norm: int = 0
    emb_f16: int = 0
    untied: int = 0

    @classmethod
    def bitnet_2b(cls, max_ctx: int = 4096) -> "DecoderConfig":
        """ModelConfig::bitnet_2b_default (config.rs:155-177)."""
        return cls(30, 2560, 20, 5, 128, 6912, 128256, max_ctx, 1e-5, 500000.0)

    @classmethod
    def falcon3(cls, n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx, rms_eps=1e-5,
                rope_theta=100000.0) -> "DecoderConfig":
        """The Falcon3 architecture (ModelConfig::falcon3_*_default, config.rs:179-227)."""
        return cls(n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx, rms_eps, rope_theta,
                   ACT_SILU, ROPE_NORMAL, 1, 1, 1)

    @classmethod
    def falcon3_10b(cls, max_ctx: int = 4096, n_layers: int = 40) -> "DecoderConfig":
        """BASELINE.json configs[1]'s Falcon3-10B shapes (40 layers, hidden 3072, 12 / 4 heads of 256, FFN 23040,
        vocabulary 131072) with the constants of falcon3_7b_default (config.rs:205-227)."""
        return cls.falcon3(n_layers, 3072, 12, 4, 256, 23040, 131072, max_ctx)

    @property
    def has_sub_norms(self) -> bool:
        return not self.no_sub_norm

    def projection_shape(self, kind: int) -> tuple:
        qd, kvd = self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        return {PROJ_Q: (qd, self.hidden), PROJ_K: (kvd, self.hidden), PROJ_V: (kvd, self.hidden),
                PROJ_O: (self.hidden, qd), PROJ_GATE: (self.ffn, self.hidden), PROJ_UP: (self.ffn, self.hidden),
                PROJ_DOWN: (self.hidden, self.ffn)}[kind]

    def _c(self) -> _Config:
        c = _Config()
        c.struct_size = ctypes.sizeof(_Config)
        for f in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "max_ctx", "rms_eps",
                  "rope_theta", "act", "rope_mode", "no_sub_norm", "emb_f16", "untied"):
            setattr(c, f, getattr(self, f))
        return c


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class Decoder:
    """A model resident on the GPU with its KV cache; step() is forward_token, generate() the greedy loop."""

    def __init__(self, config: DecoderConfig):
        self.config = config
        h = ctypes.c_void_p()
        check(lib().vx_decoder_create(ctypes.byref(config._c()), ctypes.byref(h)))
        self.handle = h

    def set_projection(self, layer: int, kind: int, planar, weight_scale: float) -> None:
        p = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
        check(lib().vx_decoder_set_projection(self.handle, layer, kind, _ptr(p), p.size, weight_scale))

    def adopt_projection(self, layer: int, kind: int, matrix) -> None:
        """vx_decoder_adopt_projection: the decoder takes over a VelurexHipLayer's matrix (the layer object is emptied)."""
        check(lib().vx_decoder_adopt_projection(self.handle, layer, kind, matrix._h))
        matrix._h = ctypes.c_void_p()

    def set_norm(self, layer: int, kind: int, weights) -> None:
        w = np.ascontiguousarray(weights, dtype=np.float32).reshape(-1)
        check(lib().vx_decoder_set_norm(self.handle, layer, kind, _ptr(w), w.size))

    def set_embedding_bf16(self, emb_bits) -> None:
        e = np.ascontiguousarray(emb_bits, dtype=np.uint16).reshape(-1)
        check(lib().vx_decoder_set_embedding_bf16(self.handle, _ptr(e), e.size))

    def set_embedding_f16(self, emb_bits) -> None:
        e = np.ascontiguousarray(emb_bits, dtype=np.uint16).reshape(-1)
        check(lib().vx_decoder_set_embedding_f16(self.handle, _ptr(e), e.size))

    def set_embedding(self, emb_bits) -> None:
        """The embedding in the config's type (f16 when emb_f16, else bf16)."""
        (self.set_embedding_f16 if self.config.emb_f16 else self.set_embedding_bf16)(emb_bits)

    def set_head(self, head_bits) -> None:
        """The untied head (vocab x hidden, the embedding's type)."""
        h = np.ascontiguousarray(head_bits, dtype=np.uint16).reshape(-1)
        check(lib().vx_decoder_set_head(self.handle, _ptr(h), h.size))

    def step(self, token: int, pos: int, want_logits: bool = True):
        """forward_token: (logits as float32 array or None, greedy next token)."""
        logits = np.empty(self.config.vocab, dtype=np.float32) if want_logits else None
        nxt = ctypes.c_uint32()
        check(lib().vx_decoder_step(self.handle, token, pos, _ptr(logits) if want_logits else None,
                                    logits.size if want_logits else 0, ctypes.byref(nxt)))
        return logits, int(nxt.value)

    def generate(self, prompt, n_new: int, stepwise: bool = False) -> list:
        """Greedy generation from position 0: the prompt by prefill passes (vx_decoder_generate), or one decode step
        per prompt token as the reference feeds it (stepwise, vx_decoder_generate_stepwise)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32).reshape(-1)
        out = np.zeros(max(n_new, 1), dtype=np.uint32)
        fn = lib().vx_decoder_generate_stepwise if stepwise else lib().vx_decoder_generate
        check(fn(self.handle, _ptr(p), p.size, n_new, _ptr(out), out.size))
        return [int(t) for t in out[:n_new]]

    def prefill(self, tokens, pos0: int = 0, want_logits: bool = True):
        """vx_decoder_prefill: tokens at positions pos0 .. into the KV cache; (logits of the last position, its greedy
        next token)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        logits = np.empty(self.config.vocab, dtype=np.float32) if want_logits else None
        nxt = ctypes.c_uint32()
        check(lib().vx_decoder_prefill(self.handle, _ptr(t), t.size, pos0, _ptr(logits) if want_logits else None,
                                       logits.size if want_logits else 0, ctypes.byref(nxt)))
        return logits, int(nxt.value)

    def kv(self, layer: int, pos: int, kv_head: int):
        """The cached f16 key and value bits (uint16 arrays of head_dim) of (layer, pos, kv_head)."""
        k = np.empty(self.config.head_dim, np.uint16)
        v = np.empty(self.config.head_dim, np.uint16)
        check(lib().vx_decoder_kv_get(self.handle, layer, pos, kv_head, _ptr(k), _ptr(v), k.size))
        return k, v

    def memory_bytes(self) -> int:
        b = ctypes.c_size_t()
        check(lib().vx_decoder_memory_bytes(self.handle, ctypes.byref(b)))
        return b.value

    def norm_fallbacks(self) -> int:
        """Workgroups on this GPU whose RMSNorm took the reference's sequential order (a diagnostic counter)."""
        c = ctypes.c_uint64()
        check(lib().vx_decoder_norm_fallbacks(self.handle, ctypes.byref(c)))
        return c.value

    def close(self) -> None:
        if self.handle:
            check(lib().vx_decoder_free(self.handle))
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuOptions(ctypes.Structure):
    """vx_gpu_options_t (quintrit_gpu_options_t): device, context limit (0 = min(4096, the model's maximum)), flags."""
    _fields_ = [("struct_size", ctypes.c_uint32), ("device_index", ctypes.c_uint32), ("context_length", ctypes.c_uint32),
                ("flags", ctypes.c_uint32)]


def open_gguf(path, context_length: int = 0, device_index: int = 0) -> Decoder:
    """quintrit_model_open_gpu (quintrit.h:527): a GGUF model (I2_S BitNet / Falcon3 / LLaMA-style) as a Decoder, parsed,
    checked and converted by vx_decoder_open_gguf."""
    o = GpuOptions(ctypes.sizeof(GpuOptions), device_index, context_length, 0)
    h = ctypes.c_void_p()
    check(lib().vx_decoder_open_gguf(str(path).encode(), ctypes.byref(o), ctypes.byref(h)))
    c = _Config()
    c.struct_size = ctypes.sizeof(_Config)
    st = lib().vx_decoder_config(h, ctypes.byref(c))
    if st != 0:
        lib().vx_decoder_free(h)
        check(st)
    dec = Decoder.__new__(Decoder)
    dec.config = DecoderConfig(*(getattr(c, f) for f, _ in _Config._fields_[1:]))
    dec.handle = h
    return dec
