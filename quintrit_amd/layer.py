"""Host-side mirror of the reference's projection-layer interface for the velurex GEMV on MI355X.

``VelurexHipLayer`` has the methods of ``TernaryGemvLayer`` (quintrit-runtime/src/layer.rs:72-87): ``forward``,
``kernel_type``, ``memory_bytes``, ``shape`` and ``weight_scale``, with the same argument meaning and the same
epilogue (layer.rs:246-253). Weights live in HBM behind a ``vx_matrix_t`` handle of libvelurex_hip.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

KERNEL_TYPE = "VelurexHip"  # the TernaryKernelType id a Rust binding would add (layer.rs:13-32)
BPW = 1.6                     # TernaryKernelType::bpw (layer.rs:62-68)
ACTIVATION_QUANT_LEVELS = 127.0  # TernaryKernelType::activation_quant_levels (layer.rs:51-60)


class VelurexHipLayer:
    """A ternary projection whose weights are resident in GPU memory."""

    def __init__(self, planar: np.ndarray, rows: int, cols: int, weight_scale: float):
        """``planar``: the reference's planar velurex bytes (quintrit-core/src/pack.rs:103-131), rows x
        ceil(cols/160)*32 bytes."""
        buf = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
        handle = ctypes.c_void_p()
        L = _lib.lib()
        _lib.check(L.vx_matrix_create(buf.ctypes.data_as(ctypes.c_void_p), buf.size, rows, cols,
                                      ctypes.c_float(weight_scale), ctypes.byref(handle)))
        self._h = handle
        self._rows = rows
        self._cols = cols

    @classmethod
    def _from_handle(cls, handle: ctypes.c_void_p) -> "VelurexHipLayer":
        """Takes ownership of a matrix handle created elsewhere (vx_gguf_upload_matrix, vx_matrix_create_ggml_dev)."""
        self = cls.__new__(cls)
        self._h = handle
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(_lib.lib().vx_matrix_shape(handle, ctypes.byref(r), ctypes.byref(c)))
        self._rows, self._cols = r.value, c.value
        return self

    def close(self) -> None:
        if self._h:
            _lib.check(_lib.lib().vx_matrix_free(self._h))
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    # ---- TernaryGemvLayer ---------------------------------------------------------------------------------------------

    def forward(self, activations: np.ndarray, act_scale: float, out: np.ndarray) -> None:
        """y = alpha * beta * (W x) into ``out`` (float32, ``rows`` values); host arrays (layer.rs:74)."""
        a = np.ascontiguousarray(activations, dtype=np.int8)
        if a.size != self._cols:
            raise ValueError(f"activations hold {a.size} values, cols = {self._cols}")
        if out.dtype != np.float32 or not out.flags.c_contiguous or out.size != self._rows:
            raise ValueError("out must be a contiguous float32 array of rows values")
        _lib.check(_lib.lib().vx_layer_forward(self._h, a.ctypes.data_as(ctypes.c_void_p), a.size,
                                               ctypes.c_float(act_scale), out.ctypes.data_as(ctypes.c_void_p),
                                               out.size))

    def kernel_type(self) -> str:
        return KERNEL_TYPE

    def memory_bytes(self) -> int:
        n = ctypes.c_size_t()
        _lib.check(_lib.lib().vx_matrix_memory_bytes(self._h, ctypes.byref(n)))
        return n.value

    def shape(self) -> tuple:
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(_lib.lib().vx_matrix_shape(self._h, ctypes.byref(r), ctypes.byref(c)))
        return (r.value, c.value)

    def weight_scale(self) -> float:
        s = ctypes.c_float()
        _lib.check(_lib.lib().vx_matrix_weight_scale(self._h, ctypes.byref(s)))
        return s.value

    # ---- device-memory entry points (torch tensors on the GPU) ----------------------------------------------------------

    def gemv_i32(self, acts_dev, out_dev, stream=None) -> None:
        """Exact int32 GEMV of device tensors (torch int8 [cols] -> int32 [rows]), enqueued on ``stream``."""
        _lib.check(_lib.lib().vx_gemv_i32_dev(self._h, ctypes.c_void_p(acts_dev.data_ptr()), acts_dev.numel(),
                                              ctypes.c_void_p(out_dev.data_ptr()), out_dev.numel(),
                                              _stream_ptr(stream)))

    def gemv_f32(self, acts_dev, act_scale: float, out_dev, stream=None) -> None:
        _lib.check(_lib.lib().vx_gemv_f32_dev(self._h, ctypes.c_void_p(acts_dev.data_ptr()), acts_dev.numel(),
                                              ctypes.c_float(act_scale), ctypes.c_void_p(out_dev.data_ptr()),
                                              out_dev.numel(), _stream_ptr(stream)))

    def gemv_lut_i32(self, lut_dev, out_dev, stream=None) -> None:
        """The int32 GEMV through compact activation tables (torch int8 tensor built by compact_lut_dev for this
        layer's cols) -> int32 [rows]; the same results as gemv_i32 on the same activations."""
        _lib.check(_lib.lib().vx_gemv_lut_i32_dev(self._h, ctypes.c_void_p(lut_dev.data_ptr()), lut_dev.numel(),
                                                  ctypes.c_void_p(out_dev.data_ptr()), out_dev.numel(),
                                                  _stream_ptr(stream)))

    def gemv_lut_f32(self, lut_dev, act_scale: float, out_dev, stream=None) -> None:
        _lib.check(_lib.lib().vx_gemv_lut_f32_dev(self._h, ctypes.c_void_p(lut_dev.data_ptr()), lut_dev.numel(),
                                                  ctypes.c_float(act_scale), ctypes.c_void_p(out_dev.data_ptr()),
                                                  out_dev.numel(), _stream_ptr(stream)))


def compact_lut(acts_dev, cols: int, stream=None):
    """The compact activation tables (vx_compact_lut_dev) of int8 device activations as a new int8 device tensor."""
    import torch
    lut = torch.empty(_lib.compact_lut_bytes(cols), dtype=torch.int8, device=acts_dev.device)
    _lib.compact_lut_dev(acts_dev.data_ptr(), acts_dev.numel(), cols, lut.data_ptr(), lut.numel(), _stream_ptr(stream))
    return lut


def _stream_ptr(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def gemv_planar_i32(planar: np.ndarray, rows: int, cols: int, acts: np.ndarray) -> np.ndarray:
    """One-shot host GEMV with quintrit_gemv_i32's argument meaning (quintrit.h:208-210)."""
    w = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty(rows, np.int32)
    _lib.check(_lib.lib().vx_gemv_planar_i32(w.ctypes.data_as(ctypes.c_void_p), w.size, rows, cols,
                                             a.ctypes.data_as(ctypes.c_void_p), a.size,
                                             out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out


def gemv_planar_f32(planar: np.ndarray, rows: int, cols: int, acts: np.ndarray, scale: float) -> np.ndarray:
    w = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
    a = np.ascontiguousarray(acts, dtype=np.int8)
    out = np.empty(rows, np.float32)
    _lib.check(_lib.lib().vx_gemv_planar_f32(w.ctypes.data_as(ctypes.c_void_p), w.size, rows, cols,
                                             a.ctypes.data_as(ctypes.c_void_p), a.size, ctypes.c_float(scale),
                                             out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out
