"""Selection policy for WKV backends.

Mirrors src/rwkv7m/kernels/wkv_backend.py:52-86 of the reference: an
explicit request wins, then the ``RWKV7M_WKV_BACKEND`` environment variable,
then ``auto`` (cpu -> reference, tpu -> pallas_tpu, gpu -> a Pallas GPU
lowering chosen by device kind). ``ffi`` is never chosen automatically, so
the HIP kernels are used exactly when a caller registers them and selects
``ffi`` -- the reference's drop-in route for a native backend.
"""

from __future__ import annotations

import os
from typing import Literal, cast

WKVBackend = Literal[
    "reference",
    "pallas_tpu",
    "pallas_gpu_mosaic",
    "pallas_gpu_triton",
    "ffi",
]

_BACKENDS = frozenset(
    {"reference", "pallas_tpu", "pallas_gpu_mosaic", "pallas_gpu_triton",
     "ffi"}
)
_HOPPER_OR_NEWER_MARKERS = (
    "h100", "h200", "gh200", "b100", "b200", "gb200", "blackwell",
)


def available_wkv_backends() -> tuple[str, ...]:
    """Return backend names accepted by the dispatcher."""
    return tuple(sorted(_BACKENDS))


def _default_platform() -> str:
    import torch

    return "gpu" if torch.cuda.is_available() else "cpu"


def _default_device_kind() -> str:
    import torch

    if not torch.cuda.is_available():
        return ""
    return str(torch.cuda.get_device_name(0)).lower()


def resolve_wkv_backend(requested: str | None = None, *,
                        platform: str | None = None,
                        device_kind: str | None = None) -> WKVBackend:
    """Resolve an explicit or automatic WKV backend (reference policy)."""
    selected = requested
    if selected is None:
        selected = os.environ.get("RWKV7M_WKV_BACKEND", "auto")
    selected = selected.strip().lower()
    if selected != "auto":
        if selected not in _BACKENDS:
            choices = ", ".join(("auto", *sorted(_BACKENDS)))
            raise ValueError(
                f"unknown WKV backend {selected!r}; expected one of {choices}"
            )
        return cast(WKVBackend, selected)

    current_platform = platform or _default_platform()
    if current_platform == "tpu":
        return "pallas_tpu"
    if current_platform == "gpu":
        kind = (device_kind or _default_device_kind()).lower()
        if any(marker in kind for marker in _HOPPER_OR_NEWER_MARKERS):
            return "pallas_gpu_mosaic"
        return "pallas_gpu_triton"
    return "reference"


__all__ = ["WKVBackend", "available_wkv_backends", "resolve_wkv_backend"]
