"""velurex ternary GEMV decode path on AMD Instinct MI355X (gfx950).

The compute lives in libvelurex_hip.so (C ABI: include/velurex_hip.h); this package is its Python host side.
"""
from ._lib import VxError, device_count, layout, lib  # noqa: F401
from .layer import VelurexHipLayer, gemv_planar_f32, gemv_planar_i32  # noqa: F401

__version__ = "0.1.0"
