"""HIP (gfx950) WKV-7 backend: ctypes binding of librwkv7m_wkv.so.

This is the native implementation that plugs into the reference's FFI
registry (src/rwkv7m/kernels/wkv_ffi.py:21-67). Its three callables have the
reference's signatures and return conventions:

* ``forward(r, w, k, v, neg_kk, kka, S0) -> (y, S_T)``
* ``forward_with_aux(...) -> ((y, S_T), aux)`` with
  ``aux = (checkpoints, interval)``: checkpoints
  ``[ceil(T/ci)+1, B, H, N, N]`` (entry 0 = S0, entry c = state after token
  ``c*ci - 1``, last = S_T; the layout of wkv_pallas_gpu.py:83-120) in the
  library's checkpoint dtype (bf16 for bf16 vectors with N = 64 and an
  interval of 16, 32 or 64, else fp32) and the interval as a 0-d int64 CPU
  tensor.
* ``backward(r, w, k, v, neg_kk, kka, S0, dy, dS_T, *aux)`` -> seven input
  cotangents in primal order and primal dtypes.

Vectors are time-major ``[T, B, H, N]`` (the reference's layout contract,
src/rwkv7m/model/wkv.py:19-57). ``layout="bthn"`` on forward,
forward_with_aux and backward takes batch-major ``[B, T, H, N]`` vectors
instead (the model's own activation layout, which the reference transposes
around every call at src/rwkv7m/model/nnx_model.py:695-698 and :709-711);
states and checkpoints keep their layouts, and the outputs follow the
vectors' layout.

Tensors are torch device tensors (torch supplies device memory and the
current HIP stream; the kernels and every check of shapes and dtypes live in
the C library). There is no CPU fallback: a missing library, a CPU tensor or
a failed launch raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

from .wkv_ffi import WKVFFIBackend, register_wkv_ffi_backend

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "librwkv7m_wkv.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1

# Every symbol declared in include/rwkv7m_wkv.h, include/rwkv7m_timemix.h
# and include/rwkv7m_screening.h.
EXPORTED_SYMBOLS = (
    "rwkv7m_abi_version",
    "rwkv7m_last_error",
    "rwkv7m_device_status",
    "rwkv7m_debug_set_wait_limit",
    "rwkv7m_debug_set_backward_segments",
    "rwkv7m_debug_set_forward_segments",
    "rwkv7m_wkv7_last_path",
    "rwkv7m_wkv7_checkpoint_count",
    "rwkv7m_wkv7_default_checkpoint_interval",
    "rwkv7m_wkv7_checkpoint_dtype",
    "rwkv7m_wkv7_forward",
    "rwkv7m_wkv7_forward_with_aux",
    "rwkv7m_wkv7_backward",
    "rwkv7m_wkv7_forward_bthn",
    "rwkv7m_wkv7_forward_with_aux_bthn",
    "rwkv7m_wkv7_backward_bthn",
    "rwkv7m_wkv7_decode_inplace",
    "rwkv7m_timemix_workspace_floats",
    "rwkv7m_timemix_wkv_inputs",
    "rwkv7m_timemix_wkv_inputs_backward",
    "rwkv7m_timemix_wkv_output",
    "rwkv7m_timemix_wkv_output_backward",
    "rwkv7m_timemix_wkv_output_backward_noalloc",
    "rwkv7m_timemix_wkv_backward",
    "rwkv7m_screen_slot_scan_workspace_floats",
    "rwkv7m_screen_slot_scan",
    "rwkv7m_screen_slot_scan_backward",
    "rwkv7m_screen_read",
    "rwkv7m_screen_read_backward",
    "rwkv7m_screen_write",
    "rwkv7m_screen_write_backward",
)

LAYOUTS = ("tbhn", "bthn")

_lib = None
_lock = threading.Lock()


def load_library(path: str | None = None):
    """Load librwkv7m_wkv.so and declare its signatures.

    Raises ``RuntimeError`` if the library has not been built.
    """
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"HIP WKV library not found at {p}; build it with "
                "`python -m rwkv7m_amd._build` (or __graft_entry__.build())")
        lib = ctypes.CDLL(p)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        lib.rwkv7m_abi_version.restype = i32
        lib.rwkv7m_abi_version.argtypes = []
        lib.rwkv7m_last_error.restype = ctypes.c_char_p
        lib.rwkv7m_last_error.argtypes = []
        lib.rwkv7m_device_status.restype = i32
        lib.rwkv7m_device_status.argtypes = [vp]
        lib.rwkv7m_debug_set_wait_limit.restype = None
        lib.rwkv7m_debug_set_wait_limit.argtypes = [i64]
        lib.rwkv7m_debug_set_backward_segments.restype = None
        lib.rwkv7m_debug_set_backward_segments.argtypes = [i32]
        lib.rwkv7m_debug_set_forward_segments.restype = None
        lib.rwkv7m_debug_set_forward_segments.argtypes = [i32]
        lib.rwkv7m_wkv7_last_path.restype = ctypes.c_char_p
        lib.rwkv7m_wkv7_last_path.argtypes = []
        lib.rwkv7m_wkv7_checkpoint_count.restype = i64
        lib.rwkv7m_wkv7_checkpoint_count.argtypes = [i64, i64]
        lib.rwkv7m_wkv7_default_checkpoint_interval.restype = i64
        lib.rwkv7m_wkv7_default_checkpoint_interval.argtypes = [i32, i64]
        lib.rwkv7m_wkv7_checkpoint_dtype.restype = i32
        lib.rwkv7m_wkv7_checkpoint_dtype.argtypes = [i32, i64, i64]
        for sfx in ("", "_bthn"):
            fwd = getattr(lib, "rwkv7m_wkv7_forward" + sfx)
            fwd.restype = i32
            fwd.argtypes = [i32] + [i64] * 4 + [vp] * 10
            aux = getattr(lib, "rwkv7m_wkv7_forward_with_aux" + sfx)
            aux.restype = i32
            aux.argtypes = [i32] + [i64] * 4 + [vp] * 10 + [i64, vp]
            bwd = getattr(lib, "rwkv7m_wkv7_backward" + sfx)
            bwd.restype = i32
            bwd.argtypes = [i32] + [i64] * 4 + [vp] * 10 + [i64] + [vp] * 8
        lib.rwkv7m_wkv7_decode_inplace.restype = i32
        lib.rwkv7m_wkv7_decode_inplace.argtypes = [i32] + [i64] * 3 + [vp] * 9
        f64 = ctypes.c_double
        dims = [i32, i64, i64, i64]
        lib.rwkv7m_timemix_workspace_floats.restype = i64
        lib.rwkv7m_timemix_workspace_floats.argtypes = [i64] * 3
        lib.rwkv7m_timemix_wkv_inputs.restype = i32
        lib.rwkv7m_timemix_wkv_inputs.argtypes = dims + [vp] * 10
        lib.rwkv7m_timemix_wkv_inputs_backward.restype = i32
        lib.rwkv7m_timemix_wkv_inputs_backward.argtypes = (
            dims + [vp] * 16 + [i64, vp])
        lib.rwkv7m_timemix_wkv_output.restype = i32
        lib.rwkv7m_timemix_wkv_output.argtypes = dims + [vp] * 8 + [f64,
                                                                    vp, vp]
        lib.rwkv7m_timemix_wkv_output_backward.restype = i32
        lib.rwkv7m_timemix_wkv_output_backward.argtypes = (
            dims + [vp] * 8 + [f64] + [vp] * 10 + [i64, vp])
        lib.rwkv7m_timemix_wkv_output_backward_noalloc.restype = i32
        lib.rwkv7m_timemix_wkv_output_backward_noalloc.argtypes = (
            dims + [vp] * 8 + [f64] + [vp] * 9 + [vp])
        lib.rwkv7m_timemix_wkv_backward.restype = i32
        lib.rwkv7m_timemix_wkv_backward.argtypes = (
            [i32] + [i64] * 4 + [vp] * 10 + [i64] + [vp] * 11)
        sdims = [i32, i64, i64, i64, i64]
        lib.rwkv7m_screen_slot_scan_workspace_floats.restype = i64
        lib.rwkv7m_screen_slot_scan_workspace_floats.argtypes = [i64] * 4
        lib.rwkv7m_screen_slot_scan.restype = i32
        lib.rwkv7m_screen_slot_scan.argtypes = sdims + [vp] * 8 + [i64, vp]
        lib.rwkv7m_screen_slot_scan_backward.restype = i32
        lib.rwkv7m_screen_slot_scan_backward.argtypes = (
            sdims + [vp] * 10 + [i64, vp])
        rdims = [i32, i64, i64, i64, i64, i64, vp, vp, vp, f64, vp, i32,
                 i32, i32, f64, f64, f64, f64]
        lib.rwkv7m_screen_read.restype = i32
        lib.rwkv7m_screen_read.argtypes = rdims + [vp] * 5
        lib.rwkv7m_screen_read_backward.restype = i32
        lib.rwkv7m_screen_read_backward.argtypes = rdims + [vp] * 7
        wdims = [i32] + [i64] * 5 + [vp] * 7 + [f64, f64]
        lib.rwkv7m_screen_write.restype = i32
        lib.rwkv7m_screen_write.argtypes = wdims + [vp] * 10
        lib.rwkv7m_screen_write_backward.restype = i32
        lib.rwkv7m_screen_write_backward.argtypes = wdims + [vp] * 15
        if path is None:
            _lib = lib
        return lib


def _check(rc: int, fn: str) -> None:
    if rc != 0:
        msg = load_library().rwkv7m_last_error().decode()
        raise RuntimeError(f"{fn} failed (status {rc}): {msg}")


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"WKV vectors must be bfloat16 or float32, got {t.dtype}")


def _dev(tensors) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "the HIP WKV backend needs GPU tensors; got a tensor on "
                f"{t.device} (there is no CPU fallback)")
        if t.device != dev:
            raise RuntimeError("all WKV tensors must be on one device")
    return dev


def _p(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _vecs(r, w, k, v, neg_kk, kka):
    out = tuple(x.contiguous() for x in (r, w, k, v, neg_kk, kka))
    if out[0].dim() != 4:
        raise ValueError(f"r must have shape [time, batch, heads, head_size]"
                         f" (or [batch, time, ...]), got {tuple(out[0].shape)}")
    # the kernels take bare pointers: every vector must have r's shape and
    # dtype, or they would read past a shorter one
    for x, name in zip(out[1:], ("w", "k", "v", "neg_kk", "kka")):
        if x.shape != out[0].shape or x.dtype != out[0].dtype:
            raise ValueError(f"{name} has shape {tuple(x.shape)} and dtype "
                             f"{x.dtype}; expected {tuple(out[0].shape)} "
                             f"{out[0].dtype} like r")
    return out


def _state(s, shape, name):
    """A contiguous fp32 state of ``shape`` ([B, H, N, N]) or raise."""
    if tuple(s.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(s.shape)}; expected "
                         f"{tuple(shape)}")
    if s.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {s.dtype}")
    return s.contiguous()


def _layout(layout: str, r: torch.Tensor):
    """(entry-point suffix, T, B, H, N) of vectors in ``layout``."""
    if layout == "tbhn":
        T, B, H, N = r.shape
        return "", T, B, H, N
    if layout == "bthn":
        B, T, H, N = r.shape
        return "_bthn", T, B, H, N
    raise ValueError(f"layout must be one of {LAYOUTS}, got {layout!r}")


def last_path() -> str:
    """Kernel path of the last successful WKV-7 call on this thread
    ("wave_forward", "decode", "seq_forward", "wave_backward",
    "seq_backward" or "")."""
    return load_library().rwkv7m_wkv7_last_path().decode()


def device_status(device=None) -> None:
    """Synchronise the device's current stream and raise ``RuntimeError`` if
    any bounded wait inside the kernels gave up since the last check (the
    affected outputs are NaN); clears the device's failure count."""
    dev = torch.device(device) if device is not None else \
        torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(dev):
        rc = load_library().rwkv7m_device_status(_stream(dev))
    _check(rc, "rwkv7m_device_status")


def set_wait_limit(polls: int) -> None:
    """Poll budget of the kernels' bounded waits for later launches (0: the
    library default).  For tests of the failure path."""
    load_library().rwkv7m_debug_set_wait_limit(int(polls))


def set_backward_segments(workgroups_per_head: int) -> None:
    """Workgroups per head of the MFMA backward for later launches (0: as
    many as the idle CUs allow).  Results are bit-identical for every count;
    for tests."""
    load_library().rwkv7m_debug_set_backward_segments(int(workgroups_per_head))


def set_forward_segments(workgroups_per_head: int) -> None:
    """Workgroups per head of the MFMA forward for later launches (0: as
    many as the idle CUs allow).  Results are bit-identical for every count;
    for tests."""
    load_library().rwkv7m_debug_set_forward_segments(int(workgroups_per_head))


def default_checkpoint_interval(dtype: torch.dtype, head_size: int) -> int:
    code = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F32
    return int(load_library().rwkv7m_wkv7_default_checkpoint_interval(
        code, head_size))


def checkpoint_count(T: int, interval: int) -> int:
    return int(load_library().rwkv7m_wkv7_checkpoint_count(T, interval))


def checkpoint_dtype(dtype: torch.dtype, head_size: int,
                     interval: int) -> torch.dtype:
    """Element type of the checkpoints for these vectors and interval."""
    code = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F32
    out = int(load_library().rwkv7m_wkv7_checkpoint_dtype(
        code, head_size, interval))
    return torch.bfloat16 if out == DTYPE_BF16 else torch.float32


def forward(r, w, k, v, neg_kk, kka, initial_state, *, out_state=None,
            layout: str = "tbhn"):
    """y, S_T = WKV(...). ``out_state`` may be ``initial_state`` (in place)."""
    lib = load_library()
    r, w, k, v, a, b = _vecs(r, w, k, v, neg_kk, kka)
    sfx, T, B, H, N = _layout(layout, r)
    s0 = _state(initial_state, (B, H, N, N), "initial_state")
    y = torch.empty_like(r)
    if out_state is not None:
        if out_state.shape != s0.shape or out_state.dtype != torch.float32 \
                or not out_state.is_contiguous():
            raise ValueError("out_state must be a contiguous float32 state "
                             "like initial_state")
    s_t = out_state if out_state is not None else torch.empty_like(s0)
    dev = _dev((r, w, k, v, a, b, s0, s_t))
    fn = "rwkv7m_wkv7_forward" + sfx
    with torch.cuda.device(dev):
        rc = getattr(lib, fn)(
            _dtype_code(r), T, B, H, N, _p(r), _p(w), _p(k), _p(v), _p(a),
            _p(b), _p(s0), _p(y), _p(s_t), _stream(dev))
    _check(rc, fn)
    return y, s_t


def forward_with_aux(r, w, k, v, neg_kk, kka, initial_state, *,
                     checkpoint_interval: int = 0, layout: str = "tbhn"):
    """((y, S_T), (checkpoints, interval)) for the backward pass."""
    lib = load_library()
    r, w, k, v, a, b = _vecs(r, w, k, v, neg_kk, kka)
    sfx, T, B, H, N = _layout(layout, r)
    s0 = _state(initial_state, (B, H, N, N), "initial_state")
    dev = _dev((r, w, k, v, a, b, s0))
    ci = int(checkpoint_interval) or default_checkpoint_interval(r.dtype, N)
    nck = checkpoint_count(T, ci)
    y = torch.empty_like(r)
    s_t = torch.empty_like(s0)
    ckpt = torch.empty((nck, B, H, N, N), device=dev,
                       dtype=checkpoint_dtype(r.dtype, N, ci))
    fn = "rwkv7m_wkv7_forward_with_aux" + sfx
    with torch.cuda.device(dev):
        rc = getattr(lib, fn)(
            _dtype_code(r), T, B, H, N, _p(r), _p(w), _p(k), _p(v), _p(a),
            _p(b), _p(s0), _p(y), _p(s_t), _p(ckpt), ci, _stream(dev))
    _check(rc, fn)
    return (y, s_t), (ckpt, torch.tensor(ci, dtype=torch.int64))


def backward(r, w, k, v, neg_kk, kka, initial_state, dy, ds_t, checkpoints,
             interval, *, layout: str = "tbhn", add=None):
    """Seven input cotangents (primal order, primal dtypes).

    ``add``: ``(dr_add, dk_add, dv_add)`` (each a vector-shaped tensor or
    None), cotangents of r, k and v from their other uses, summed into dr,
    dk and dv in fp32 before rounding (``rwkv7m_timemix_wkv_backward``;
    batch-major vectors only)."""
    lib = load_library()
    r, w, k, v, a, b = _vecs(r, w, k, v, neg_kk, kka)
    sfx, T, B, H, N = _layout(layout, r)
    s0 = _state(initial_state, (B, H, N, N), "initial_state")
    dev = _dev((r, w, k, v, a, b, s0, checkpoints))
    ci = int(interval)
    if checkpoints.shape != (checkpoint_count(T, ci), B, H, N, N) or \
            checkpoints.dtype != checkpoint_dtype(r.dtype, N, ci):
        raise ValueError("checkpoints do not match time, shape and interval")
    ckpt = checkpoints.contiguous()
    if dy is not None and tuple(dy.shape) != tuple(r.shape):
        raise ValueError(f"dy has shape {tuple(dy.shape)}; expected "
                         f"{tuple(r.shape)}")
    dy_c = None if dy is None else dy.to(r.dtype).contiguous()
    ds_c = None if ds_t is None else _state(ds_t.to(torch.float32),
                                            (B, H, N, N), "ds_t")
    _dev([t for t in (r, dy_c, ds_c) if t is not None])
    grads = [torch.empty_like(r) for _ in range(6)]
    ds0 = torch.empty_like(s0)
    if add is not None:
        if layout != "bthn":
            raise ValueError("added cotangents need batch-major vectors "
                             "(layout='bthn')")
        adds = []
        for t, name in zip(add, ("dr_add", "dk_add", "dv_add")):
            if t is not None and tuple(t.shape) != tuple(r.shape):
                raise ValueError(f"{name} has shape {tuple(t.shape)}; "
                                 f"expected {tuple(r.shape)}")
            adds.append(None if t is None else t.to(r.dtype).contiguous())
        _dev([r] + [t for t in adds if t is not None])
        fn = "rwkv7m_timemix_wkv_backward"
        with torch.cuda.device(dev):
            rc = lib.rwkv7m_timemix_wkv_backward(
                _dtype_code(r), T, B, H, N, _p(r), _p(w), _p(k), _p(v),
                _p(a), _p(b), _p(s0), _p(dy_c), _p(ds_c), _p(ckpt), ci,
                *(_p(t) for t in adds), *(_p(g) for g in grads), _p(ds0),
                _stream(dev))
        _check(rc, fn)
        return (*grads, ds0)
    fn = "rwkv7m_wkv7_backward" + sfx
    with torch.cuda.device(dev):
        rc = getattr(lib, fn)(
            _dtype_code(r), T, B, H, N, _p(r), _p(w), _p(k), _p(v), _p(a),
            _p(b), _p(s0), _p(dy_c), _p(ds_c), _p(ckpt), ci,
            *(_p(g) for g in grads), _p(ds0), _stream(dev))
    _check(rc, fn)
    return (*grads, ds0)


def decode_inplace(r, w, k, v, neg_kk, kka, state):
    """One-token step, state updated in place; vectors [B,H,N] or
    [1,B,H,N]. Returns y with the vectors' shape."""
    lib = load_library()
    shape = r.shape
    r, w, k, v, a, b = _vecs(*(x.reshape(-1, *x.shape[-3:])
                               for x in (r, w, k, v, neg_kk, kka)))
    if r.shape[0] != 1 or not state.is_contiguous():
        raise ValueError("decode_inplace takes one token and a contiguous "
                         "state")
    _, B, H, N = r.shape
    if tuple(state.shape) != (B, H, N, N) or state.dtype != torch.float32:
        raise ValueError(f"state must be a float32 [{B}, {H}, {N}, {N}] "
                         f"tensor, got {state.dtype} {tuple(state.shape)}")
    dev = _dev((r, w, k, v, a, b, state))
    y = torch.empty_like(r)
    with torch.cuda.device(dev):
        rc = lib.rwkv7m_wkv7_decode_inplace(
            _dtype_code(r), B, H, N, _p(r), _p(w), _p(k), _p(v), _p(a),
            _p(b), _p(state), _p(y), _stream(dev))
    _check(rc, "rwkv7m_wkv7_decode_inplace")
    return y.reshape(shape)


def hip_wkv_ffi_backend() -> WKVFFIBackend:
    """The HIP kernels as a reference-contract ``WKVFFIBackend``."""
    load_library()
    return WKVFFIBackend(
        forward=forward,
        forward_with_aux=forward_with_aux,
        backward=lambda *args: backward(*args),
    )


def register_hip_backend(*, replace: bool = False) -> WKVFFIBackend:
    """Register the HIP kernels as the process's WKV FFI backend; select it
    with ``backend="ffi"`` or ``RWKV7M_WKV_BACKEND=ffi``."""
    backend = hip_wkv_ffi_backend()
    register_wkv_ffi_backend(backend, replace=replace)
    return backend


__all__ = [
    "EXPORTED_SYMBOLS", "LAYOUTS", "LIB_PATH", "backward", "checkpoint_count",
    "checkpoint_dtype",
    "decode_inplace", "default_checkpoint_interval", "device_status",
    "forward", "forward_with_aux", "hip_wkv_ffi_backend", "last_path",
    "load_library", "register_hip_backend", "set_wait_limit",
]
