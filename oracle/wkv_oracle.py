"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the WKV-7 recurrence.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or as the
timed CPU baseline. No product code path imports it.

Two independent restatements of the reference algorithm live here:

* ``forward`` / ``backward``: ctypes wrappers over ``wkv_oracle.c`` (plain C
  loops, float64 for parity, float32 for the CPU baseline).
* ``np_forward`` / ``np_backward``: numpy, vectorised over (batch, head),
  written separately so the two can check each other.

Reference semantics followed (paths relative to the reference repository):

* ``src/rwkv7m/model/rwkv_core.py:54-86`` -- one ``wkv_step``.
* ``src/rwkv7m/model/wkv.py:60-67`` -- ``lax.scan`` over time; ``y`` stacked
  in fp32 and cast to the vector dtype once, after the scan.
* ``src/rwkv7m/kernels/wkv_pallas_gpu.py:221-257`` -- reverse equations.
* ``src/rwkv7m/kernels/wkv_pallas_gpu.py:83-120`` -- checkpoint aux format.

Pinning (each check lives in ``tests/test_oracle.py``): the reference's numpy
known-answer test (``tests/test_upstream_rwkv7_parity.py:265-297``), closed
forms (pure decay, running outer-product sum, T=1), row independence,
float64 torch autograd of an explicit matrix-product formulation, and central
finite differences.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_wkv.so")
_lib = None
_lib_lock = threading.Lock()


def build() -> str:
    """Compile the C oracle in place (gcc via the Makefile beside it)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle_wkv.so"],
                   check=True)
    return _LIB_PATH


def _load():
    global _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                build()
            lib = ctypes.CDLL(_LIB_PATH)
            i64, vp, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
            for suffix in ("f64", "f32"):
                fwd = getattr(lib, f"oracle_wkv7_forward_{suffix}")
                fwd.argtypes = [i64] * 4 + [vp] * 10 + [i64, ci]
                fwd.restype = None
                bwd = getattr(lib, f"oracle_wkv7_backward_{suffix}")
                bwd.argtypes = [i64] * 4 + [vp] * 16 + [ci]
                bwd.restype = None
            _lib = lib
    return _lib


def _ptr(x: np.ndarray):
    return x.ctypes.data_as(ctypes.c_void_p)


def _prep(arrays, dtype):
    return [np.ascontiguousarray(np.asarray(x, dtype=np.float64), dtype=dtype)
            for x in arrays]


def forward(r, w, k, v, neg_kk, kka, s0, *, checkpoint_interval=None,
            precision="f64", threads=1):
    """Run the C oracle forward.

    Inputs are array-likes of shape ``[T,B,H,N]`` (vectors) and ``[B,H,N,N]``
    (state); they are upcast (bf16 values are exact in both precisions).
    Returns ``(y, s_t)`` or ``(y, s_t, checkpoints)`` in the chosen precision;
    ``y`` is not rounded to the vector dtype (use ``bf16_round``).
    """
    dt = np.float64 if precision == "f64" else np.float32
    r, w, k, v, a, b, s0 = _prep((r, w, k, v, neg_kk, kka, s0), dt)
    T, B, H, N = r.shape
    assert s0.shape == (B, H, N, N)
    y = np.zeros((T, B, H, N), dt)
    s_t = np.zeros((B, H, N, N), dt)
    ckpt = None
    ci = 0
    if checkpoint_interval is not None:
        ci = int(checkpoint_interval)
        ckpt = np.zeros(((T + ci - 1) // ci + 1, B, H, N, N), dt)
    fn = getattr(_load(), f"oracle_wkv7_forward_{precision}")
    fn(T, B, H, N, _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
       _ptr(s0), _ptr(y), _ptr(s_t),
       _ptr(ckpt) if ckpt is not None else None, ci, int(threads))
    if ckpt is not None:
        return y, s_t, ckpt
    return y, s_t


def backward(r, w, k, v, neg_kk, kka, s0, dy, ds_t, *, precision="f64",
             threads=1):
    """Run the C oracle reverse pass; returns the seven input cotangents
    ``(dr, dw, dk, dv, dneg_kk, dkka, ds0)`` in primal order."""
    dt = np.float64 if precision == "f64" else np.float32
    r, w, k, v, a, b, s0, dy, ds_t = _prep(
        (r, w, k, v, neg_kk, kka, s0, dy, ds_t), dt)
    T, B, H, N = r.shape
    outs = [np.zeros((T, B, H, N), dt) for _ in range(6)]
    ds0 = np.zeros((B, H, N, N), dt)
    fn = getattr(_load(), f"oracle_wkv7_backward_{precision}")
    fn(T, B, H, N, _ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
       _ptr(s0), _ptr(dy), _ptr(ds_t), *(_ptr(o) for o in outs), _ptr(ds0),
       int(threads))
    return (*outs, ds0)


# ---------------------------------------------------------------------------
# numpy restatement (independent of the C code; vectorised over (b, h))
# ---------------------------------------------------------------------------

def np_forward(r, w, k, v, neg_kk, kka, s0, *, return_states=False):
    """float64 numpy scan of ``wkv_step`` (rwkv_core.py:54-86)."""
    r, w, k, v, a, b, s = (np.asarray(x, np.float64)
                           for x in (r, w, k, v, neg_kk, kka, s0))
    s = s.copy()
    T = r.shape[0]
    ys = np.zeros(r.shape, np.float64)
    states = [s.copy()]
    sas = np.zeros(r.shape, np.float64)
    for t in range(T):
        d = np.exp(-np.exp(w[t]))                      # [B,H,N] over j
        sa = np.einsum("bhij,bhj->bhi", s, a[t])       # row-wise S @ a
        s = (s * d[..., None, :]
             + sa[..., :, None] * b[t][..., None, :]
             + v[t][..., :, None] * k[t][..., None, :])
        ys[t] = np.einsum("bhij,bhj->bhi", s, r[t])
        sas[t] = sa
        if return_states:
            states.append(s.copy())
    if return_states:
        return ys, s, np.stack(states), sas
    return ys, s


def np_backward(r, w, k, v, neg_kk, kka, s0, dy, ds_t):
    """float64 numpy reverse pass (wkv_pallas_gpu.py:221-257 equations),
    using stored states instead of division by the decay."""
    r, w, k, v, a, b = (np.asarray(x, np.float64)
                        for x in (r, w, k, v, neg_kk, kka))
    dy = np.asarray(dy, np.float64)
    _, _, states, sas = np_forward(r, w, k, v, a, b, s0, return_states=True)
    ds = np.array(ds_t, np.float64)
    T = r.shape[0]
    grads = [np.zeros(r.shape, np.float64) for _ in range(6)]
    dr, dw, dk, dv, da, db = grads
    for t in range(T - 1, -1, -1):
        sp, sc, sa = states[t], states[t + 1], sas[t]
        d = np.exp(-np.exp(w[t]))
        g = ds + dy[t][..., :, None] * r[t][..., None, :]
        dr[t] = np.einsum("bhij,bhi->bhj", sc, dy[t])
        dd = np.einsum("bhij,bhij->bhj", g, sp)
        dsa = np.einsum("bhij,bhj->bhi", g, b[t])
        db[t] = np.einsum("bhij,bhi->bhj", g, sa)
        dv[t] = np.einsum("bhij,bhj->bhi", g, k[t])
        dk[t] = np.einsum("bhij,bhi->bhj", g, v[t])
        da[t] = np.einsum("bhij,bhi->bhj", sp, dsa)
        dw[t] = dd * (-np.exp(w[t]) * d)
        ds = g * d[..., None, :] + dsa[..., :, None] * a[t][..., None, :]
    return (dr, dw, dk, dv, da, db, ds)


# ---------------------------------------------------------------------------
# bfloat16 helpers (round-to-nearest-even through uint32 bit operations)
# ---------------------------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """float -> uint16 bfloat16 bit patterns, round to nearest even."""
    f = np.ascontiguousarray(np.asarray(x, np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(f)
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out


def bf16_from_bits(bits) -> np.ndarray:
    u = np.asarray(bits, np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 value, returned as float32."""
    return bf16_from_bits(bf16_bits(x))


def normalized_max_error(actual, expected) -> float:
    """max|actual - expected| / max|expected| (0 if both are all-zero)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    scale = np.max(np.abs(expected)) if expected.size else 0.0
    err = np.max(np.abs(actual - expected)) if expected.size else 0.0
    if scale == 0.0:
        return float(err)
    return float(err / scale)


__all__ = [
    "backward", "bf16_bits", "bf16_from_bits", "bf16_round", "build",
    "forward", "normalized_max_error", "np_backward", "np_forward",
]
