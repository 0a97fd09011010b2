"""TEST INFRASTRUCTURE ONLY: float64 numpy oracle of the fused time-mix
producers and consumer around the WKV call.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or as
the timed CPU baseline.  No product code path imports it.

Reference semantics (src/rwkv7m/model/nnx_model.py, NNXRWKV7TimeMix):

* ``:630`` -- ``w = -softplus(-w_raw) - 0.5``;
* ``:683-686`` -- ``kk = k * k_k`` normalised per head by
  ``sqrt(sum kk^2 + 1e-12**2)``;
* ``:687`` -- ``k' = k * (1 + (a - 1) * k_a)`` (after kk is taken);
* ``:693-694`` -- WKV's ``neg_kk = -kk`` and ``kka = kk * a``;
* ``:709-720`` with ``_group_norm`` ``:368-373`` -- flax ``GroupNorm`` over
  H groups of the N channels, statistics in fp32, epsilon ``64e-5``
  (``:559-562``), ``use_fast_variance`` (flax's default): variance
  ``max(0, E[y^2] - E[y]^2)``, then ``* scale + bias``;
* ``:721-727`` -- ``+ sum_head(r * k' * r_k) * v``, then ``* g``.

The backward functions are the vector-Jacobian products of those
expressions (the reference differentiates them with jax autodiff).

Activations are ``[rows, C]`` float64 (C = H * N); parameters ``[C]``.

Pinning (``tests/test_oracle.py``): library routines on the same inputs
(torch.nn.functional softplus / normalize / group_norm in float64), the
invariants unit head norm and zero-mean, unit-variance GroupNorm, the
asymptotes of the clamp, and central finite differences plus float64 torch
autograd for every backward output.
"""

from __future__ import annotations

import numpy as np

KK_EPS = 1e-12  # nnx_model.py:686, squared inside the square root


def _heads(x, N):
    rows, C = x.shape
    return x.reshape(rows, C // N, N)


def wkv_inputs(w_raw, k, a, k_k, k_a, N):
    """(w, k', neg_kk, kka) -- nnx_model.py:630, :683-694."""
    w = -np.logaddexp(-w_raw, 0.0) - 0.5
    kk0 = _heads(k * k_k, N)
    nrm = np.sqrt((kk0 * kk0).sum(-1, keepdims=True) + KK_EPS ** 2)
    kk = (kk0 / nrm).reshape(k.shape)
    kp = k * (1.0 + (a - 1.0) * k_a)
    return w, kp, -kk, kk * a


def wkv_inputs_backward(w_raw, k, a, k_k, k_a, dw, dkp, dneg_kk, dkka, N):
    """(dw_raw, dk, da, dk_k, dk_a): VJP of ``wkv_inputs``."""
    dw_raw = dw / (1.0 + np.exp(w_raw))  # d/dx (-softplus(-x)) = sigmoid(-x)
    kk0 = _heads(k * k_k, N)
    nrm = np.sqrt((kk0 * kk0).sum(-1, keepdims=True) + KK_EPS ** 2)
    kk = kk0 / nrm
    g_kk = _heads(dkka * a - dneg_kk, N)
    dkk0 = ((g_kk - kk * (g_kk * kk).sum(-1, keepdims=True)) / nrm
            ).reshape(k.shape)
    kk = kk.reshape(k.shape)
    scale = 1.0 + (a - 1.0) * k_a
    dk = dkk0 * k_k + dkp * scale
    da = dkka * kk + dkp * k * k_a
    dk_k = (dkk0 * k).sum(0)
    dk_a = (dkp * k * (a - 1.0)).sum(0)
    return dw_raw, dk, da, dk_k, dk_a


def _group_norm(y, scale, bias, N, eps):
    yh = _heads(y, N)
    mean = yh.mean(-1, keepdims=True)
    var = np.maximum(0.0, (yh * yh).mean(-1, keepdims=True) - mean * mean)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (yh - mean) * rstd
    return (xhat.reshape(y.shape) * scale + bias, xhat.reshape(y.shape),
            rstd)


def wkv_output(y, r, k, v, g, r_k, scale, bias, N, eps=64e-5):
    """(GroupNorm(y) + sum_head(r k r_k) v) * g -- nnx_model.py:709-727."""
    gn, _, _ = _group_norm(y, scale, bias, N, eps)
    s = _heads(r * k * r_k, N).sum(-1, keepdims=True)
    bonus = (s * _heads(v, N)).reshape(y.shape)
    return (gn + bonus) * g


def wkv_output_backward(y, r, k, v, g, r_k, scale, bias, dout, N,
                        eps=64e-5):
    """(dy, dr, dk, dv, dg, dr_k, dscale, dbias): VJP of ``wkv_output``."""
    gn, xhat, rstd = _group_norm(y, scale, bias, N, eps)
    s = _heads(r * k * r_k, N).sum(-1, keepdims=True)
    z = gn + (s * _heads(v, N)).reshape(y.shape)
    dg = dout * z
    dz = dout * g
    dv = (_heads(dz, N) * s).reshape(y.shape)
    ds = _heads(dz * v, N).sum(-1, keepdims=True)
    dr = (ds * _heads(k * r_k, N)).reshape(y.shape)
    dk = (ds * _heads(r * r_k, N)).reshape(y.shape)
    dr_k = (ds * _heads(r * k, N)).reshape(y.shape).sum(0)
    dscale = (dz * xhat).sum(0)
    dbias = dz.sum(0)
    dxh = _heads(dz * scale, N)
    xh = _heads(xhat, N)
    dy = (rstd * (dxh - dxh.mean(-1, keepdims=True)
                  - xh * (dxh * xh).mean(-1, keepdims=True))).reshape(y.shape)
    return dy, dr, dk, dv, dg, dr_k, dscale, dbias
