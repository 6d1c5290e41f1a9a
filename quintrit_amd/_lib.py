"""ctypes binding of libvelurex_hip.so (include/velurex_hip.h).

The library is the product: there is no CPU fallback. Importing a compute entry point without the built library, or
calling one without a gfx950 GPU, raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvelurex_hip.so")

VX_OK = 0
STATUS_NAMES = {
    0: "VX_OK", 1: "VX_ERR_NULL_POINTER", 2: "VX_ERR_INVALID_ARGUMENT", 3: "VX_ERR_INVALID_SHAPE",
    4: "VX_ERR_BUFFER_TOO_SMALL", 5: "VX_ERR_INVALID_VALUE", 6: "VX_ERR_UNSUPPORTED", 7: "VX_ERR_IO",
    8: "VX_ERR_FORMAT", 9: "VX_ERR_NOT_FOUND", 10: "VX_ERR_MODEL", 11: "VX_ERR_CONTEXT_OVERFLOW",
    12: "VX_ERR_BUSY", 13: "VX_ERR_INTERNAL", 14: "VX_ERR_INVALID_HANDLE", 15: "VX_ERR_DEVICE",
}


class VxError(RuntimeError):
    """A vx_* call returned a status other than VX_OK."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class _Layout(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("tile_rows", ctypes.c_uint32), ("tile_group", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("rows", ctypes.c_uint64),
                ("cols", ctypes.c_uint64), ("padded_rows", ctypes.c_uint64), ("planar_row_bytes", ctypes.c_uint64),
                ("tile_row_bytes", ctypes.c_uint64), ("device_row_bytes", ctypes.c_uint64),
                ("device_bytes", ctypes.c_uint64)]


_lib = None

# name -> (restype, argtypes); every symbol include/velurex_hip.h declares.
_vp, _sz, _f32, _i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int
SIGNATURES = {
    "vx_status_string": (ctypes.c_char_p, [_i32]),
    "vx_last_error_code": (_i32, []),
    "vx_last_error_message": (ctypes.c_char_p, []),
    "vx_version": (ctypes.c_char_p, []),
    "vx_abi_version": (ctypes.c_uint32, []),
    "vx_device_count": (_i32, [_vp]),
    "vx_layout": (_i32, [_sz, _sz, _vp]),
    "vx_device_layout_pack": (_i32, [_vp, _sz, _sz, _sz, _vp, _sz]),
    "vx_matrix_create": (_i32, [_vp, _sz, _sz, _sz, _f32, _vp]),
    "vx_matrix_create_dev": (_i32, [_vp, _sz, _sz, _sz, _f32, _vp]),
    "vx_matrix_free": (_i32, [_vp]),
    "vx_matrix_shape": (_i32, [_vp, _vp, _vp]),
    "vx_matrix_memory_bytes": (_i32, [_vp, _vp]),
    "vx_matrix_weight_scale": (_i32, [_vp, _vp]),
    "vx_matrix_device_weights": (_i32, [_vp, _vp]),
    "vx_gemv_i32_dev": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "vx_gemv_f32_dev": (_i32, [_vp, _vp, _sz, _f32, _vp, _sz, _vp]),
    "vx_staged_bytes": (_i32, [_sz, _vp]),
    "vx_stage_acts_dev": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "vx_gemv_staged_i32_dev": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "vx_gemv_staged_f32_dev": (_i32, [_vp, _vp, _sz, _f32, _vp, _sz, _vp]),
    "vx_compact_lut_bytes": (_i32, [_sz, _vp]),
    "vx_compact_lut_dev": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "vx_gemv_lut_i32_dev": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "vx_gemv_lut_f32_dev": (_i32, [_vp, _vp, _sz, _f32, _vp, _sz, _vp]),
    "vx_layer_forward": (_i32, [_vp, _vp, _sz, _f32, _vp, _sz]),
    "vx_gemv_planar_i32": (_i32, [_vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz]),
    "vx_gemv_planar_f32": (_i32, [_vp, _sz, _sz, _sz, _vp, _sz, _f32, _vp, _sz]),
    "vx_plan_create": (_i32, [_vp, _sz, _vp]),
    "vx_lut_plan_create": (_i32, [_vp, _sz, _vp]),
    "vx_plan_run": (_i32, [_vp, _vp]),
    "vx_plan_work_items": (_i32, [_vp, _vp]),
    "vx_plan_free": (_i32, [_vp]),
    "vx_gemm_workspace_bytes": (_i32, [_vp, _sz, _vp]),
    "vx_gemm_i32_dev": (_i32, [_vp, _vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp]),
    "vx_gemm_i32_noalloc_dev": (_i32, [_vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "vx_q2_matrix_create": (_i32, [_vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    "vx_q2_gemv_f32_dev": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp]),
    "vx_q2_lane_sums_dev": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "vx_q2_plan_create": (_i32, [_vp, _sz, _vp]),
    "vx_decoder_create": (_i32, [_vp, _vp]),
    "vx_decoder_set_projection": (_i32, [_vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _sz, _f32]),
    "vx_decoder_set_norm": (_i32, [_vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _sz]),
    "vx_decoder_set_embedding_bf16": (_i32, [_vp, _vp, _sz]),
    "vx_decoder_set_embedding_f16": (_i32, [_vp, _vp, _sz]),
    "vx_decoder_set_head": (_i32, [_vp, _vp, _sz]),
    "vx_decoder_step": (_i32, [_vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _sz, _vp]),
    "vx_decoder_generate": (_i32, [_vp, _vp, _sz, _sz, _vp, _sz]),
    "vx_decoder_generate_stepwise": (_i32, [_vp, _vp, _sz, _sz, _vp, _sz]),
    "vx_decoder_prefill": (_i32, [_vp, _vp, _sz, ctypes.c_uint32, _vp, _sz, _vp]),
    "vx_decoder_kv_get": (_i32, [_vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _vp, _vp, _sz]),
    "vx_decoder_memory_bytes": (_i32, [_vp, _vp]),
    "vx_decoder_norm_fallbacks": (_i32, [_vp, _vp]),
    "vx_decoder_config": (_i32, [_vp, _vp]),
    "vx_decoder_adopt_projection": (_i32, [_vp, ctypes.c_uint32, ctypes.c_uint32, _vp]),
    "vx_decoder_open_gguf": (_i32, [ctypes.c_char_p, _vp, _vp]),
    "vx_decoder_free": (_i32, [_vp]),
    "vx_expf_dev": (_i32, [_vp, _sz, _vp, _vp]),
    "vx_gguf_open": (_i32, [ctypes.c_char_p, _vp]),
    "vx_gguf_close": (_i32, [_vp]),
    "vx_gguf_info": (_i32, [_vp, _vp]),
    "vx_gguf_tensor_at": (_i32, [_vp, _sz, _vp]),
    "vx_gguf_tensor_find": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_gguf_metadata_string": (_i32, [_vp, ctypes.c_char_p, _vp, _sz, _vp]),
    "vx_gguf_metadata_u64": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_gguf_metadata_f64": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_gguf_metadata_json": (_i32, [_vp, _vp, _sz, _vp]),
    "vx_gguf_tensor_data": (_i32, [_vp, ctypes.c_char_p, _vp, _vp]),
    "vx_gguf_tensor_scale": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_gguf_convert_planar": (_i32, [_vp, ctypes.c_char_p, _vp, _sz, _vp, _vp, _vp]),
    "vx_ggml_to_planar": (_i32, [ctypes.c_int32, _vp, _sz, _sz, _sz, _vp, _sz]),
    "vx_gguf_upload_matrix": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_gguf_convert_q2_0": (_i32, [_vp, ctypes.c_char_p, _vp, _sz, _vp, _sz, _vp, _vp]),
    "vx_gguf_upload_q2_matrix": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "vx_matrix_create_ggml_dev": (_i32, [ctypes.c_int32, _vp, _sz, _sz, _sz, _f32, _vp]),
}


def lib() -> ctypes.CDLL:
    """Loads the HIP library; raises if it was not built (there is no fallback)."""
    global _lib
    if _lib is None:
        try:  # one HIP runtime per process: torch's, when torch is present (it is matched by soname)
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (or make -C "
                               f"quintrit_amd/csrc); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != VX_OK:
        msg = lib().vx_last_error_message()
        raise VxError(status, msg.decode() if msg else "")


def layout(rows: int, cols: int) -> dict:
    lay = _Layout()
    lay.struct_size = ctypes.sizeof(_Layout)
    check(lib().vx_layout(rows, cols, ctypes.byref(lay)))
    return {name: getattr(lay, name) for name, _ in _Layout._fields_ if name not in ("struct_size", "reserved")}


def device_layout_pack(planar, rows: int, cols: int):
    """Host conversion of planar bytes into the device layout (vx_device_layout_pack)."""
    import numpy as np
    p = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
    n = layout(rows, cols)["device_bytes"]
    out = np.empty(n, np.uint8)
    check(lib().vx_device_layout_pack(p.ctypes.data_as(ctypes.c_void_p), p.size, rows, cols,
                                      out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out


def staged_bytes(cols: int) -> int:
    n = ctypes.c_size_t()
    check(lib().vx_staged_bytes(cols, ctypes.byref(n)))
    return n.value


def device_count() -> int:
    n = ctypes.c_int32()
    check(lib().vx_device_count(ctypes.byref(n)))
    return n.value


class GemvJob(ctypes.Structure):
    """vx_gemv_job_t (include/velurex_hip.h)."""
    _fields_ = [("struct_size", ctypes.c_uint32), ("out_f32", ctypes.c_int32), ("matrix", ctypes.c_void_p),
                ("staged", ctypes.c_void_p), ("staged_len", ctypes.c_size_t), ("act_scale_dev", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("out_capacity", ctypes.c_size_t), ("acts", ctypes.c_void_p)]


class Plan:
    """A batched GEMV plan (vx_plan_t): many GEMVs in one persistent launch."""

    def __init__(self, jobs):
        arr = (GemvJob * len(jobs))()
        for i, j in enumerate(jobs):
            arr[i] = j
            if not arr[i].struct_size:  # a caller may give the older, shorter size (no acts field)
                arr[i].struct_size = ctypes.sizeof(GemvJob)
        h = ctypes.c_void_p()
        check(lib().vx_plan_create(arr, len(jobs), ctypes.byref(h)))
        self._h = h

    def run(self, stream_ptr) -> None:
        check(lib().vx_plan_run(self._h, stream_ptr))

    def work_items(self) -> int:
        n = ctypes.c_uint32()
        check(lib().vx_plan_work_items(self._h, ctypes.byref(n)))
        return n.value

    def close(self) -> None:
        if self._h:
            check(lib().vx_plan_free(self._h))
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LutPlan(Plan):
    """A plan of GEMVs through the compact activation tables (vx_lut_plan_create): each job's `staged` is the table
    set of its matrix's cols (compact_lut_dev); run and freed like Plan."""

    def __init__(self, jobs):  # noqa: super().__init__ builds digit-table plans
        arr = (GemvJob * len(jobs))()
        for i, j in enumerate(jobs):
            arr[i] = j
            arr[i].struct_size = ctypes.sizeof(GemvJob)
        h = ctypes.c_void_p()
        check(lib().vx_lut_plan_create(arr, len(jobs), ctypes.byref(h)))
        self._h = h


def compact_lut_bytes(cols: int) -> int:
    n = ctypes.c_size_t()
    check(lib().vx_compact_lut_bytes(cols, ctypes.byref(n)))
    return n.value


def compact_lut_dev(acts_ptr: int, acts_len: int, cols: int, lut_ptr: int, lut_capacity: int, stream_ptr=None) -> None:
    """Builds the compact activation tables of `cols` int8 activations at acts_ptr into lut_ptr (device pointers)."""
    check(lib().vx_compact_lut_dev(ctypes.c_void_p(acts_ptr), acts_len, cols, ctypes.c_void_p(lut_ptr), lut_capacity,
                                   stream_ptr))


class Q2Job(ctypes.Structure):
    """vx_q2_job_t (include/velurex_hip.h)."""
    _fields_ = [("struct_size", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("matrix", ctypes.c_void_p),
                ("acts", ctypes.c_void_p), ("acts_len", ctypes.c_size_t), ("act_scales", ctypes.c_void_p),
                ("n_act_scales", ctypes.c_size_t), ("out", ctypes.c_void_p), ("out_capacity", ctypes.c_size_t)]


class Q2Plan(Plan):
    """A plan of Q2_0 GEMVs (vx_q2_plan_create), run and freed like Plan."""

    def __init__(self, jobs):  # noqa: super().__init__ builds velurex plans
        arr = (Q2Job * len(jobs))()
        for i, j in enumerate(jobs):
            arr[i] = j
            arr[i].struct_size = ctypes.sizeof(Q2Job)
        h = ctypes.c_void_p()
        check(lib().vx_q2_plan_create(arr, len(jobs), ctypes.byref(h)))
        self._h = h


class Q2Matrix:
    """A Q2_0 matrix in GPU memory (vx_q2_matrix_create): planar trits + fp16 scales, one per 64 weights."""

    def __init__(self, planar, scales_f16, rows: int, cols: int):
        import numpy as np
        p = np.ascontiguousarray(planar, dtype=np.uint8).reshape(-1)
        s = np.ascontiguousarray(scales_f16, dtype=np.float16).view(np.uint16).reshape(-1)
        h = ctypes.c_void_p()
        check(lib().vx_q2_matrix_create(p.ctypes.data_as(ctypes.c_void_p), p.size, s.ctypes.data_as(ctypes.c_void_p),
                                        s.size, rows, cols, ctypes.byref(h)))
        self.handle, self.rows, self.cols = h, rows, cols

    @classmethod
    def _from_handle(cls, handle, rows: int, cols: int) -> "Q2Matrix":
        m = cls.__new__(cls)
        m.handle, m.rows, m.cols = handle, rows, cols
        return m

    def gemv_f32(self, acts_dev, act_scales_dev, out_dev, stream_ptr) -> None:
        check(lib().vx_q2_gemv_f32_dev(self.handle, ctypes.c_void_p(acts_dev.data_ptr()), acts_dev.numel(),
                                       ctypes.c_void_p(act_scales_dev.data_ptr()), act_scales_dev.numel(),
                                       ctypes.c_void_p(out_dev.data_ptr()), out_dev.numel(), stream_ptr))

    def lane_sums(self, acts_dev, out_dev, stream_ptr) -> None:
        check(lib().vx_q2_lane_sums_dev(self.handle, ctypes.c_void_p(acts_dev.data_ptr()), acts_dev.numel(),
                                        ctypes.c_void_p(out_dev.data_ptr()), out_dev.numel(), stream_ptr))

    def close(self) -> None:
        if self.handle:
            check(lib().vx_matrix_free(self.handle))
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
