"""WKV backends and the native-backend registry (mirrors rwkv7m.kernels,
src/rwkv7m/kernels/__init__.py:1-21, plus the HIP backend)."""

from .wkv_backend import WKVBackend, available_wkv_backends, resolve_wkv_backend
from .wkv_ffi import (
    WKVFFIBackend,
    register_wkv_ffi_backend,
    require_wkv_ffi_backend,
    unregister_wkv_ffi_backend,
)
from .wkv_hip import hip_wkv_ffi_backend, register_hip_backend

__all__ = [
    "WKVBackend",
    "WKVFFIBackend",
    "available_wkv_backends",
    "hip_wkv_ffi_backend",
    "register_hip_backend",
    "register_wkv_ffi_backend",
    "require_wkv_ffi_backend",
    "resolve_wkv_backend",
    "unregister_wkv_ffi_backend",
]
