"""rwkv7m_amd: MI355X-native (gfx950) WKV-7 recurrence, forward and backward.

The public surface mirrors the reference's WKV path (``rwkv7m.model.wkv`` and
``rwkv7m.kernels``): ``wkv7``, ``wkv7_reference``, the backend policy and the
FFI registry. The hand-written HIP kernels live in ``librwkv7m_wkv.so``
(C ABI in ``include/rwkv7m_wkv.h``) and are used after
``register_hip_backend()`` with ``backend="ffi"`` or
``RWKV7M_WKV_BACKEND=ffi``.  ``time_mix_wkv``, ``wkv7_inputs`` and
``wkv7_output`` are the fused HIP producers and consumer around the call in
the time mix (C ABI in ``include/rwkv7m_timemix.h``).
"""

from .kernels import (
    WKVBackend,
    WKVFFIBackend,
    available_wkv_backends,
    hip_wkv_ffi_backend,
    register_hip_backend,
    register_wkv_ffi_backend,
    require_wkv_ffi_backend,
    resolve_wkv_backend,
    unregister_wkv_ffi_backend,
)
from .timemix import time_mix_wkv, wkv7_inputs, wkv7_output
from .wkv import wkv7, wkv7_batch_major, wkv7_reference

__all__ = [
    "WKVBackend",
    "WKVFFIBackend",
    "available_wkv_backends",
    "hip_wkv_ffi_backend",
    "register_hip_backend",
    "register_wkv_ffi_backend",
    "require_wkv_ffi_backend",
    "resolve_wkv_backend",
    "time_mix_wkv",
    "unregister_wkv_ffi_backend",
    "wkv7",
    "wkv7_batch_major",
    "wkv7_inputs",
    "wkv7_output",
    "wkv7_reference",
]
