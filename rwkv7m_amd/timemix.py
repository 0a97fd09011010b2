"""Fused WKV input producers and output consumer of the RWKV-7 time mix.

The reference's ``NNXRWKV7TimeMix.__call__``
(src/rwkv7m/model/nnx_model.py:592-730) builds the six WKV vectors from its
projections, calls WKV and post-processes ``y``, as plain JAX ops that XLA
fuses and jax autodiff differentiates:

* producers (:630, :683-694): ``w = -softplus(-w_raw) - 0.5``;
  ``kk = normalize_head(k * k_k)``; ``k' = k * (1 + (a - 1) * k_a)``;
  ``neg_kk = -kk``; ``kka = kk * a``;
* the WKV call on ``[B, T, H, N]`` vectors swapped to time-major and back
  (:695-711);
* consumer (:709-727): ``GroupNorm(y)`` (``ln_x``, H groups, epsilon
  64e-5, fp32 statistics) ``+ (sum_head r * k' * r_k) * v``, times the gate
  ``g`` (the output projection that follows is a plain GEMM and stays with
  the caller).

Here each of those pieces is one HIP kernel per direction
(``kernels/timemix_hip.py``), and ``time_mix_wkv`` chains producers, the
batch-major WKV kernels and the consumer with no transpose and no
intermediate elementwise pass: in the backward the consumer's cotangents of
``r``, ``k'`` and ``v`` are summed into the WKV backward's own stores
(``rwkv7m_timemix_wkv_backward``).

Activations are batch-major ``[B, T, C]`` (C = H * N) as in the reference
model, bf16 or fp32; parameters any float dtype, their gradients returned
in that dtype and shape.  No CPU fallback: GPU tensors and the built
library are required.
"""

from __future__ import annotations

import torch

from .kernels import timemix_hip, wkv_hip

GROUPNORM_EPS = timemix_hip.GROUPNORM_EPS


def _pgrad(g: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return g.reshape(like.shape).to(like.dtype)


def _zeros_if_none(g, like):
    return torch.zeros_like(like) if g is None else g


def _head_size(C: int, n_heads: int) -> int:
    if n_heads <= 0 or C % n_heads:
        raise ValueError(f"d_model={C} must equal n_heads*head_size "
                         f"(n_heads={n_heads})")
    return C // n_heads


class _WKVInputs(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w_raw, k, a, k_k, k_a, n_heads):
        N = _head_size(w_raw.shape[-1], n_heads)
        outs = timemix_hip.inputs_forward(w_raw, k, a, k_k, k_a, N)
        ctx.save_for_backward(w_raw, k, a, k_k, k_a)
        ctx.N = N
        shape = (*w_raw.shape[:-1], n_heads, N)
        return tuple(o.view(shape) for o in outs)

    @staticmethod
    def backward(ctx, dw, dkp, dnkk, dkka):
        w_raw, k, a, k_k, k_a = ctx.saved_tensors
        cots = [_zeros_if_none(c, w_raw).reshape(w_raw.shape)
                for c in (dw, dkp, dnkk, dkka)]
        dx, dk, da, dkk_p, dka_p = timemix_hip.inputs_backward(
            w_raw, k, a, k_k, k_a, *cots, ctx.N)
        return dx, dk, da, _pgrad(dkk_p, k_k), _pgrad(dka_p, k_a), None


def wkv7_inputs(w_raw, k, a, k_k, k_a, n_heads: int):
    """WKV inputs ``(w, k', neg_kk, kka)``, each ``[..., H, N]``, from the
    time mix's ``w_raw``, ``k`` and ``a`` (``[..., C]``) and the parameters
    ``k_k``, ``k_a`` (C elements).  nnx_model.py:630, :683-694."""
    return _WKVInputs.apply(w_raw, k, a, k_k, k_a, n_heads)


class _WKVOutput(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, r, k, v, g, r_k, ln_scale, ln_bias, eps):
        N = y.shape[-1]
        out = timemix_hip.output_forward(y, r, k, v, g, r_k, ln_scale,
                                         ln_bias, N, eps)
        ctx.save_for_backward(y, r, k, v, g, r_k, ln_scale, ln_bias)
        ctx.N, ctx.eps = N, eps
        return out

    @staticmethod
    def backward(ctx, dout):
        y, r, k, v, g, r_k, ln_scale, ln_bias = ctx.saved_tensors
        dout = _zeros_if_none(dout, g)
        dy, dr, dk, dv, dg, drk, dsc, dbi = timemix_hip.output_backward(
            y, r, k, v, g, r_k, ln_scale, ln_bias, dout, ctx.N, ctx.eps)
        return (dy, dr, dk, dv, dg, _pgrad(drk, r_k), _pgrad(dsc, ln_scale),
                _pgrad(dbi, ln_bias), None)


def wkv7_output(y, r, k, v, g, r_k, ln_scale, ln_bias,
                eps: float = GROUPNORM_EPS):
    """Time-mix output before the output projection:
    ``(GroupNorm(y) + (sum_head r * k * r_k) * v) * g`` with ``y, r, k, v``
    ``[..., H, N]`` (``k`` the scaled key k'), ``g`` ``[..., C]``; returns
    ``[..., C]``.  nnx_model.py:709-727."""
    if y.dim() < 2:
        raise ValueError(f"y must have shape [..., heads, head_size], got "
                         f"{tuple(y.shape)}")
    return _WKVOutput.apply(y, r, k, v, g, r_k, ln_scale, ln_bias, eps)


class _TimeMixWKV(torch.autograd.Function):
    """Producers -> batch-major WKV -> consumer as one custom VJP; the
    backward runs consumer, WKV and producer kernels in turn, with the
    consumer's cotangents of r, k' and v added inside the WKV backward."""

    @staticmethod
    def forward(ctx, r, w_raw, k, v, a, g, k_k, k_a, r_k, ln_scale, ln_bias,
                s0, n_heads, eps, with_aux):
        B, T, C = r.shape
        N = _head_size(C, n_heads)
        hv = (B, T, n_heads, N)
        w, kp, nkk, kka = (x.view(hv) for x in timemix_hip.inputs_forward(
            w_raw, k, a, k_k, k_a, N))
        r_h, v_h = r.reshape(hv), v.reshape(hv)
        vecs = (r_h, w, kp, v_h, nkk, kka, s0)
        if with_aux:
            (y, s_t), aux = wkv_hip.forward_with_aux(*vecs, layout="bthn")
        else:
            (y, s_t), aux = wkv_hip.forward(*vecs, layout="bthn"), ()
        out = timemix_hip.output_forward(y, r_h, kp, v_h, g, r_k, ln_scale,
                                         ln_bias, N, eps)
        ctx.save_for_backward(r_h, w, kp, v_h, nkk, kka, s0, y, w_raw, k, a,
                              g, k_k, k_a, r_k, ln_scale, ln_bias)
        ctx.aux, ctx.N, ctx.eps = tuple(aux), N, eps
        return out, s_t

    @staticmethod
    def backward(ctx, dout, ds_t):
        (r_h, w, kp, v_h, nkk, kka, s0, y, w_raw, k, a, g, k_k, k_a, r_k,
         ln_scale, ln_bias) = ctx.saved_tensors
        aux, N, eps = ctx.aux, ctx.N, ctx.eps
        ctx.aux = None
        if not aux:
            raise RuntimeError("time_mix_wkv: backward needs the forward "
                               "run with gradients enabled")
        dout = _zeros_if_none(dout, g)
        ds_t = _zeros_if_none(ds_t, s0)
        dy, dr_c, dk_c, dv_c, dg, drk, dsc, dbi = timemix_hip.output_backward(
            y, r_h, kp, v_h, g, r_k, ln_scale, ln_bias, dout, N, eps)
        dr, dw, dk_w, dv, dnkk, dkka, ds0 = wkv_hip.backward(
            r_h, w, kp, v_h, nkk, kka, s0, dy, ds_t, *aux, layout="bthn",
            add=(dr_c.view(r_h.shape), dk_c.view(r_h.shape),
                 dv_c.view(r_h.shape)))
        dx, dk, da, dkk_p, dka_p = timemix_hip.inputs_backward(
            w_raw, k, a, k_k, k_a, dw, dk_w, dnkk, dkka, N)
        dr = dr.reshape(w_raw.shape)
        dv = dv.reshape(w_raw.shape)
        return (dr, dx, dk, dv, da, dg, _pgrad(dkk_p, k_k),
                _pgrad(dka_p, k_a), _pgrad(drk, r_k), _pgrad(dsc, ln_scale),
                _pgrad(dbi, ln_bias), ds0, None, None, None)


def time_mix_wkv(r, w_raw, k, v, a, g, k_k, k_a, r_k, ln_scale, ln_bias,
                 initial_state=None, *, n_heads: int,
                 eps: float = GROUPNORM_EPS):
    """The WKV section of the RWKV-7 time mix on batch-major activations.

    ``r, w_raw, k, v, a, g``: ``[B, T, C]`` (``r`` the receptance, ``w_raw``
    the decay pre-activation ``w0 + tanh(x_w w1) w2``, ``k`` the key
    projection, ``v`` the value after the v-first mix, ``a`` the in-context
    learning rate after its sigmoid, ``g`` the gate); parameters ``k_k``,
    ``k_a``, ``ln_scale``, ``ln_bias`` (C elements) and ``r_k`` (``[H,
    N]``); ``initial_state`` ``[B, H, N, N]`` fp32 (zeros if None).

    Returns ``(out [B, T, C], final_state [B, H, N, N] fp32)`` where
    ``out`` feeds the output projection: nnx_model.py:630-727 minus the
    projections.
    """
    if r.dim() != 3:
        raise ValueError(f"r must have shape [batch, time, d_model], got "
                         f"{tuple(r.shape)}")
    B, T, C = r.shape
    N = _head_size(C, n_heads)
    for name, x in (("w_raw", w_raw), ("k", k), ("v", v), ("a", a),
                    ("g", g)):
        if tuple(x.shape) != (B, T, C):
            raise ValueError(f"{name} must have shape {(B, T, C)}, got "
                             f"{tuple(x.shape)}")
        if x.dtype != r.dtype:
            raise TypeError(f"all time-mix activations must use {r.dtype}, "
                            f"got {name}={x.dtype}")
    if initial_state is None:
        initial_state = torch.zeros(B, n_heads, N, N, dtype=torch.float32,
                                    device=r.device)
    inputs = (r, w_raw, k, v, a, g, k_k, k_a, r_k, ln_scale, ln_bias,
              initial_state)
    with_aux = torch.is_grad_enabled() and any(
        isinstance(x, torch.Tensor) and x.requires_grad for x in inputs)
    return _TimeMixWKV.apply(*inputs, n_heads, eps, with_aux)


__all__ = ["GROUPNORM_EPS", "time_mix_wkv", "wkv7_inputs", "wkv7_output"]
