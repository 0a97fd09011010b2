"""WKV-7 operator API: validation, custom VJP and backend dispatch.

A torch mirror of the reference's ``src/rwkv7m/model/wkv.py``:

* ``_validate_wkv_inputs`` -- wkv.py:19-57, same exception types and messages;
* ``wkv7_reference`` -- wkv.py:60-79, the portable time-major scan of
  ``wkv_step`` (rwkv_core.py:54-86) written with torch ops;
* ``wkv7`` -- wkv.py:219-286, a custom-VJP op (``torch.autograd.Function``)
  with the same positional signature ``(r, w, k, v, neg_kk, kka,
  initial_state, backend=None, interpret=False)``, dispatching to the
  registered FFI backend (the HIP kernels once ``register_hip_backend()`` ran)
  or to the reference scan;
* ``_wkv7_forward_dispatch`` / ``_wkv7_backward_dispatch`` -- wkv.py:127-216,
  including the FFI argument order ``backward(*inputs, *cotangents, *aux)``;
* ``wkv7_batch_major`` -- the call as the reference's time-mix layer makes it
  on its batch-major activations (nnx_model.py:695-698, :709-711), without
  materialising the transposes when the HIP kernels serve it.

Layout: vectors ``[T, B, H, N]`` (bf16 or fp32, one dtype), state
``[B, H, N, N]`` fp32; ``y`` in the vector dtype, the final state fp32.
Only reverse-mode differentiation is supported (``torch.func.jvp`` raises).
"""

from __future__ import annotations

import torch

from .kernels.wkv_backend import resolve_wkv_backend
from .kernels.wkv_ffi import require_wkv_ffi_backend

_SUPPORTED_INPUT_DTYPES = (torch.bfloat16, torch.float32)


def _validate_wkv_inputs(r, w, k, v, neg_kk, kka, initial_state):
    vectors = {"r": r, "w": w, "k": k, "v": v, "neg_kk": neg_kk, "kka": kka}
    if initial_state.dim() != 4:
        raise ValueError(
            "initial_state must have shape [batch, heads, rows, columns]"
        )
    if initial_state.shape[-1] != initial_state.shape[-2]:
        raise ValueError("initial_state WKV rows and columns must be equal")
    if initial_state.dtype != torch.float32:
        raise TypeError(
            f"initial_state must be float32, got {initial_state.dtype}"
        )
    if r.dim() != 4:
        raise ValueError(
            "r must have shape [time, batch, heads, head_size], "
            f"got {tuple(r.shape)}"
        )
    expected_shape = (r.shape[0], *initial_state.shape[:3])
    for name, value in vectors.items():
        if value.dim() != 4 or tuple(value.shape) != expected_shape:
            raise ValueError(
                f"{name} must have shape {expected_shape}, "
                f"got {tuple(value.shape)}"
            )
        if value.dtype != r.dtype:
            raise TypeError(
                f"all WKV vectors must use {r.dtype}, got {name}={value.dtype}"
            )
    if r.dtype not in _SUPPORTED_INPUT_DTYPES:
        raise TypeError(
            f"WKV vectors must be bfloat16 or float32, got {r.dtype}"
        )


def _wkv7_reference_impl(r, w, k, v, neg_kk, kka, initial_state):
    """Time-major scan of the fp32 step (rwkv_core.py:54-86); ``y`` is cast
    to the vector dtype once, after the scan (wkv.py:62-67)."""
    state = initial_state.to(torch.float32)
    ys = []
    for t in range(r.shape[0]):
        r_t, w_t, k_t, v_t, a_t, b_t = (
            x[t].to(torch.float32) for x in (r, w, k, v, neg_kk, kka))
        decay = torch.exp(-torch.exp(w_t))[..., None, :]
        sa = (state * a_t[..., None, :]).sum(-1)
        state = (state * decay + sa[..., :, None] * b_t[..., None, :]
                 + v_t[..., :, None] * k_t[..., None, :])
        ys.append((state * r_t[..., None, :]).sum(-1))
    if ys:
        y = torch.stack(ys)
    else:
        y = torch.zeros(r.shape, dtype=torch.float32, device=r.device)
    return y.to(r.dtype), state


def wkv7_reference(r, w, k, v, neg_kk, kka, initial_state):
    """Execute the portable time-major WKV recurrence (wkv.py:70-79)."""
    _validate_wkv_inputs(r, w, k, v, neg_kk, kka, initial_state)
    return _wkv7_reference_impl(r, w, k, v, neg_kk, kka, initial_state)


_PALLAS = ("pallas_gpu_mosaic", "pallas_gpu_triton", "pallas_tpu")


def _no_pallas(selected: str):
    raise NotImplementedError(
        f"WKV backend {selected!r} is a JAX Pallas backend of the reference "
        "and is not part of rwkv7m_amd; register the HIP kernels with "
        "rwkv7m_amd.register_hip_backend() and select backend='ffi' "
        "(or RWKV7M_WKV_BACKEND=ffi)"
    )


def _wkv7_forward_dispatch(r, w, k, v, neg_kk, kka, initial_state, *,
                           backend, interpret, with_aux):
    selected = resolve_wkv_backend(backend)
    inputs = (r, w, k, v, neg_kk, kka, initial_state)
    if selected == "reference":
        outputs = _wkv7_reference_impl(*inputs)
        return (outputs, ()) if with_aux else outputs
    if selected in _PALLAS:
        _no_pallas(selected)
    ffi_backend = require_wkv_ffi_backend()
    if with_aux:
        return ffi_backend.forward_with_aux(*inputs)
    return ffi_backend.forward(*inputs)


def _wkv7_backward_dispatch(inputs, cotangents, aux, *, backend, interpret):
    selected = resolve_wkv_backend(backend)
    if selected == "reference":
        with torch.enable_grad():
            detached = [x.detach().requires_grad_(True) for x in inputs]
            outs = _wkv7_reference_impl(*detached)
            grads = torch.autograd.grad(
                outs, detached, grad_outputs=cotangents, allow_unused=True)
        return tuple(torch.zeros_like(x) if g is None else g.to(x.dtype)
                     for g, x in zip(grads, inputs))
    if selected in _PALLAS:
        _no_pallas(selected)
    ffi_backend = require_wkv_ffi_backend()
    return ffi_backend.backward(*inputs, *cotangents, *aux)


class _WKV7(torch.autograd.Function):
    """Custom VJP of wkv7 (the jax.custom_vjp of wkv.py:219-286).

    Every call goes through ``apply`` so that forward-mode transforms reach
    ``jvp`` and fail there, as jax.jvp fails on the reference's custom_vjp.
    ``with_aux`` is decided by the caller: the backward residuals (the
    backend's aux, e.g. state checkpoints) are only produced when a
    gradient can be requested.
    """

    @staticmethod
    def forward(r, w, k, v, neg_kk, kka, initial_state, backend, interpret,
                with_aux):
        inputs = (r, w, k, v, neg_kk, kka, initial_state)
        if not with_aux:
            y, final_state = _wkv7_forward_dispatch(
                *inputs, backend=backend, interpret=interpret,
                with_aux=False)
            return y, final_state, ()
        (y, final_state), aux = _wkv7_forward_dispatch(
            *inputs, backend=backend, interpret=interpret, with_aux=True)
        return y, final_state, tuple(aux)

    @staticmethod
    def setup_context(ctx, inputs, output):
        *primal, backend, interpret, _ = inputs
        aux = output[2]
        ctx.save_for_backward(*primal)
        ctx.aux = aux
        ctx.backend = backend
        ctx.interpret = interpret

    @staticmethod
    def backward(ctx, dy, ds_t, _aux_grad=None):
        inputs = ctx.saved_tensors
        aux = ctx.aux
        ctx.aux = None
        r, s0 = inputs[0], inputs[6]
        if dy is None:
            dy = torch.zeros_like(r)
        if ds_t is None:
            ds_t = torch.zeros_like(s0)
        grads = _wkv7_backward_dispatch(
            inputs, (dy.to(r.dtype), ds_t.to(torch.float32)), aux,
            backend=ctx.backend, interpret=ctx.interpret)
        return (*grads, None, None, None)

    @staticmethod
    def jvp(ctx, *tangents):
        raise TypeError(
            "wkv7 supports reverse-mode differentiation only; forward-mode "
            "autodiff (jvp) is not implemented")


def wkv7(r, w, k, v, neg_kk, kka, initial_state, backend: str | None = None,
         interpret: bool = False):
    """Execute WKV-7 through the selected backend (wkv.py:219-250).

    ``backend`` is normally left as ``None``/``auto``; ``"ffi"`` selects the
    registered native backend (the HIP kernels after
    ``rwkv7m_amd.register_hip_backend()``). ``interpret`` is accepted for
    signature parity and only meaningful to Pallas backends.
    """
    _validate_wkv_inputs(r, w, k, v, neg_kk, kka, initial_state)
    inputs = (r, w, k, v, neg_kk, kka, initial_state)
    with_aux = torch.is_grad_enabled() and any(x.requires_grad
                                               for x in inputs)
    y, final_state, _ = _WKV7.apply(*inputs, backend, interpret, with_aux)
    return y, final_state


# ---------------------------------------------------------------------------
# Batch-major call: the model's own [B, T, H, N] activations
# ---------------------------------------------------------------------------

def _validate_batch_major(r, w, k, v, neg_kk, kka, initial_state):
    if r.dim() != 4:
        raise ValueError(
            "r must have shape [batch, time, heads, head_size], "
            f"got {tuple(r.shape)}"
        )
    # the time-major checks on views with the first two axes swapped
    swapped = [x.transpose(0, 1) if x.dim() >= 2 else x
               for x in (r, w, k, v, neg_kk, kka)]
    try:
        _validate_wkv_inputs(*swapped, initial_state)
    except ValueError as exc:
        expected = (initial_state.shape[0], r.shape[1],
                    *initial_state.shape[1:3])
        raise ValueError(
            f"batch-major WKV vectors must all have shape {expected} "
            f"[batch, time, heads, head_size]: {exc}") from exc


class _WKV7BatchMajor(torch.autograd.Function):
    """Custom VJP of the batch-major call on the HIP kernels: forward,
    forward_with_aux and backward with ``layout="bthn"``, so no transposed
    copy of the vectors, y or the vector gradients is ever made."""

    @staticmethod
    def forward(r, w, k, v, neg_kk, kka, initial_state, with_aux):
        from .kernels import wkv_hip
        inputs = (r, w, k, v, neg_kk, kka, initial_state)
        if not with_aux:
            y, final_state = wkv_hip.forward(*inputs, layout="bthn")
            return y, final_state, ()
        (y, final_state), aux = wkv_hip.forward_with_aux(*inputs,
                                                         layout="bthn")
        return y, final_state, tuple(aux)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(*inputs[:7])
        ctx.aux = output[2]

    @staticmethod
    def backward(ctx, dy, ds_t, _aux_grad=None):
        from .kernels import wkv_hip
        inputs = ctx.saved_tensors
        aux = ctx.aux
        ctx.aux = None
        grads = wkv_hip.backward(*inputs, dy, ds_t, *aux, layout="bthn")
        return (*grads, None)

    @staticmethod
    def jvp(ctx, *tangents):
        raise TypeError(
            "wkv7 supports reverse-mode differentiation only; forward-mode "
            "autodiff (jvp) is not implemented")


def _hip_backend_registered() -> bool:
    from .kernels import wkv_ffi, wkv_hip
    backend = wkv_ffi._registered_backend
    return backend is not None and backend.forward is wkv_hip.forward


def wkv7_batch_major(r, w, k, v, neg_kk, kka, initial_state,
                     backend: str | None = None, interpret: bool = False):
    """WKV-7 on batch-major vectors ``[B, T, H, N]``; ``y`` is batch-major,
    the states ``[B, H, N, N]`` fp32 as in ``wkv7``.

    Equal to swapping the first two axes of the six vectors, calling
    ``wkv7`` and swapping ``y`` back -- what the reference's time-mix layer
    does around every call (src/rwkv7m/model/nnx_model.py:695-698,
    :709-711).  With the HIP backend registered and selected, the kernels
    read and write the batch-major tensors directly (the library's
    ``_bthn`` entry points) and the transposes are never materialised; any
    other backend runs behind the transposes.
    """
    _validate_batch_major(r, w, k, v, neg_kk, kka, initial_state)
    selected = resolve_wkv_backend(backend)
    if selected == "ffi" and _hip_backend_registered():
        inputs = (r, w, k, v, neg_kk, kka, initial_state)
        with_aux = torch.is_grad_enabled() and any(x.requires_grad
                                                   for x in inputs)
        y, final_state, _ = _WKV7BatchMajor.apply(*inputs, with_aux)
        return y, final_state
    swapped = [x.transpose(0, 1) for x in (r, w, k, v, neg_kk, kka)]
    y, final_state = wkv7(*swapped, initial_state, backend, interpret)
    return y.transpose(0, 1), final_state


__all__ = ["wkv7", "wkv7_batch_major", "wkv7_reference"]
