"""Registrable FFI boundary for native WKV implementations.

Mirrors the reference's plugin API, src/rwkv7m/kernels/wkv_ffi.py:21-67:
a frozen dataclass of three callables and a process-global registry that
rejects accidental replacement. The HIP backend of this package
(``rwkv7m_amd.kernels.wkv_hip``) is one such implementation; it is never
selected automatically.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

WKVForward = Callable[..., tuple[object, object]]
WKVForwardWithAux = Callable[
    ..., tuple[tuple[object, object], tuple[object, ...]]
]
WKVBackward = Callable[..., tuple[object, ...]]


@dataclass(frozen=True)
class WKVFFIBackend:
    """Callable contract of a native WKV extension.

    ``forward`` receives the six vectors and the initial state and returns
    ``(activation, final_state)``. ``forward_with_aux`` returns that pair plus
    an auxiliary tuple. ``backward`` receives the seven primal inputs, the two
    output cotangents, then the unpacked auxiliary tuple, and returns the
    seven input cotangents in primal order and primal dtypes.
    """

    forward: WKVForward
    forward_with_aux: WKVForwardWithAux
    backward: WKVBackward


# Process-global and not thread-safe, like the reference registry.
_registered_backend: WKVFFIBackend | None = None


def register_wkv_ffi_backend(backend: WKVFFIBackend, *,
                             replace: bool = False) -> None:
    """Register a native backend, rejecting accidental replacement."""
    global _registered_backend
    if _registered_backend is not None and not replace:
        raise RuntimeError("a WKV FFI backend is already registered")
    _registered_backend = backend


def unregister_wkv_ffi_backend() -> None:
    """Remove the process-local FFI backend registration."""
    global _registered_backend
    _registered_backend = None


def require_wkv_ffi_backend() -> WKVFFIBackend:
    """Return the registered backend or fail before any work is enqueued."""
    if _registered_backend is None:
        raise RuntimeError(
            "WKV backend 'ffi' was requested, but no FFI backend is registered"
        )
    return _registered_backend


__all__ = [
    "WKVFFIBackend",
    "register_wkv_ffi_backend",
    "require_wkv_ffi_backend",
    "unregister_wkv_ffi_backend",
]
