"""HIP (gfx950) fused producers and consumer of the time mix's WKV call:
ctypes binding of the ``rwkv7m_timemix_*`` entry points of librwkv7m_wkv.so
(include/rwkv7m_timemix.h).

The reference computes these inline in ``NNXRWKV7TimeMix.__call__``
(src/rwkv7m/model/nnx_model.py:630 and :683-694 for the producers,
:709-727 for the consumer) and differentiates them with jax autodiff; here
each direction is one kernel pass over the activations.

Activations have any shape whose element count is ``rows * C`` (C = H * N,
the last axis or the last two axes ``[H, N]``); they are read as
``[rows][C]`` contiguous, and outputs take the shape of the first
activation argument.  Parameters (k_k, k_a, r_k, ln_x scale and bias) may
have any shape of C elements (the reference's ``[1, 1, C]`` and ``[H, N]``)
and any float dtype: they are passed to the kernels as fp32 and their
gradients come back as fp32 ``[C]``.  There is no CPU fallback.
"""

from __future__ import annotations

import torch

from . import wkv_hip

GROUPNORM_EPS = 64e-5  # ln_x epsilon, nnx_model.py:559-562


def _acts(*ts):
    out = []
    for t in ts:
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
        out.append(t)
    return out


def _param(p: torch.Tensor, C: int, name: str) -> torch.Tensor:
    if p.numel() != C:
        raise ValueError(f"{name} must have {C} elements (H*N), got shape "
                         f"{tuple(p.shape)}")
    return p.detach().reshape(C).to(torch.float32).contiguous()


def _rows(x: torch.Tensor, C: int, others, names) -> int:
    if x.numel() % C:
        raise ValueError(f"activation of shape {tuple(x.shape)} is not a "
                         f"whole number of rows of C={C} channels")
    for t, n in zip(others, names):
        if t.numel() != x.numel():
            raise ValueError(f"{n} has shape {tuple(t.shape)}; expected "
                             f"{x.numel()} elements like {tuple(x.shape)}")
        if t.dtype != x.dtype:
            raise TypeError(f"{n} has dtype {t.dtype}; all activations must "
                            f"share one dtype ({x.dtype})")
    return x.numel() // C


def _heads(C: int, head_size: int) -> int:
    if head_size <= 0 or C % head_size:
        raise ValueError(f"C={C} is not a multiple of head_size={head_size}")
    return C // head_size


def _call(fn: str, *args) -> None:
    lib = wkv_hip.load_library()
    wkv_hip._check(getattr(lib, fn)(*args), fn)


def workspace_floats(rows: int, n_heads: int, head_size: int) -> int:
    n = wkv_hip.load_library().rwkv7m_timemix_workspace_floats(
        rows, n_heads, head_size)
    if n < 0:
        raise ValueError(f"invalid time-mix sizes rows={rows} H={n_heads} "
                         f"N={head_size}")
    return n


def inputs_forward(w_raw, k, a, k_k, k_a, head_size: int):
    """(w, k', neg_kk, kka) from (w_raw, k, a); shapes follow ``w_raw``."""
    C = k_k.numel()
    H = _heads(C, head_size)
    rows = _rows(w_raw, C, (k, a), ("k", "a"))
    dev = wkv_hip._dev([w_raw, k, a, k_k, k_a])
    w_raw, k, a = _acts(w_raw, k, a)
    pk, pa = _param(k_k, C, "k_k"), _param(k_a, C, "k_a")
    outs = [torch.empty_like(w_raw) for _ in range(4)]
    P = wkv_hip._p
    _call("rwkv7m_timemix_wkv_inputs", wkv_hip._dtype_code(w_raw), rows, H,
          head_size, P(w_raw), P(k), P(a), P(pk), P(pa), *map(P, outs),
          wkv_hip._stream(dev))
    return tuple(outs)


def inputs_backward(w_raw, k, a, k_k, k_a, dw, dk_out, dneg_kk, dkka,
                    head_size: int, dk_out2=None):
    """Cotangents (dw_raw, dk, da, dk_k, dk_a) of the producers; dk_out2,
    if given, is a second cotangent of k' added to dk_out.  dk_k and dk_a
    are fp32 ``[C]``."""
    C = k_k.numel()
    H = _heads(C, head_size)
    extra = (dk_out2,) if dk_out2 is not None else ()
    rows = _rows(w_raw, C, (k, a, dw, dk_out, dneg_kk, dkka) + extra,
                 ("k", "a", "dw", "dk_out", "dneg_kk", "dkka", "dk_out2"))
    dev = wkv_hip._dev([w_raw, k, a, k_k, k_a, dw, dk_out, dneg_kk, dkka,
                        *extra])
    w_raw, k, a, dw, dk_out, dneg_kk, dkka = _acts(w_raw, k, a, dw, dk_out,
                                                   dneg_kk, dkka)
    dk_out2 = _acts(dk_out2)[0] if dk_out2 is not None else None
    pk, pa = _param(k_k, C, "k_k"), _param(k_a, C, "k_a")
    grads = [torch.empty_like(w_raw) for _ in range(3)]
    pgrads = [torch.empty(C, dtype=torch.float32, device=dev)
              for _ in range(2)]
    nws = workspace_floats(rows, H, head_size)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
    P = wkv_hip._p
    _call("rwkv7m_timemix_wkv_inputs_backward", wkv_hip._dtype_code(w_raw),
          rows, H, head_size, P(w_raw), P(k), P(a), P(pk), P(pa), P(dw),
          P(dk_out), P(dk_out2), P(dneg_kk), P(dkka), *map(P, grads),
          *map(P, pgrads), P(ws), nws, wkv_hip._stream(dev))
    return (*grads, *pgrads)


def output_forward(y, r, k, v, g, r_k, ln_scale, ln_bias, head_size: int,
                   eps: float = GROUPNORM_EPS):
    """(GroupNorm(y) + (sum_head r k r_k) v) * g; shape follows ``g``."""
    C = r_k.numel()
    H = _heads(C, head_size)
    rows = _rows(g, C, (y, r, k, v), ("y", "r", "k", "v"))
    dev = wkv_hip._dev([y, r, k, v, g, r_k, ln_scale, ln_bias])
    y, r, k, v, g = _acts(y, r, k, v, g)
    prk = _param(r_k, C, "r_k")
    psc = _param(ln_scale, C, "ln_scale")
    pbi = _param(ln_bias, C, "ln_bias")
    out = torch.empty_like(g)
    P = wkv_hip._p
    _call("rwkv7m_timemix_wkv_output", wkv_hip._dtype_code(g), rows, H,
          head_size, P(y), P(r), P(k), P(v), P(g), P(prk), P(psc), P(pbi),
          float(eps), P(out), wkv_hip._stream(dev))
    return out


def output_backward(y, r, k, v, g, r_k, ln_scale, ln_bias, dout,
                    head_size: int, eps: float = GROUPNORM_EPS):
    """Cotangents (dy, dr, dk, dv, dg, dr_k, dln_scale, dln_bias) of the
    consumer; dy..dv take the shape of ``y``, dg that of ``g``, the
    parameter gradients are fp32 ``[C]``."""
    C = r_k.numel()
    H = _heads(C, head_size)
    rows = _rows(g, C, (y, r, k, v, dout), ("y", "r", "k", "v", "dout"))
    dev = wkv_hip._dev([y, r, k, v, g, r_k, ln_scale, ln_bias, dout])
    y, r, k, v, g, dout = _acts(y, r, k, v, g, dout)
    prk = _param(r_k, C, "r_k")
    psc = _param(ln_scale, C, "ln_scale")
    pbi = _param(ln_bias, C, "ln_bias")
    grads = [torch.empty_like(y) for _ in range(4)] + [torch.empty_like(g)]
    pgrads = [torch.empty(C, dtype=torch.float32, device=dev)
              for _ in range(3)]
    nws = workspace_floats(rows, H, head_size)
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
    P = wkv_hip._p
    _call("rwkv7m_timemix_wkv_output_backward", wkv_hip._dtype_code(g), rows,
          H, head_size, P(y), P(r), P(k), P(v), P(g), P(prk), P(psc), P(pbi),
          float(eps), P(dout), *map(P, grads), *map(P, pgrads), P(ws), nws,
          wkv_hip._stream(dev))
    return (*grads, *pgrads)


def output_backward_noalloc(y, r, k, v, g, r_k, ln_scale, ln_bias, dout,
                            head_size: int, eps: float = GROUPNORM_EPS,
                            out=None):
    """``output_backward`` through the entry point that allocates nothing
    on the device: the partial rows go to the library's built-in scratch.
    ``out`` (optional) holds the eight result tensors to write, so that the
    call itself allocates nothing either; calls overlapping on one device
    race on the scratch."""
    C = r_k.numel()
    H = _heads(C, head_size)
    rows = _rows(g, C, (y, r, k, v, dout), ("y", "r", "k", "v", "dout"))
    dev = wkv_hip._dev([y, r, k, v, g, r_k, ln_scale, ln_bias, dout])
    y, r, k, v, g, dout = _acts(y, r, k, v, g, dout)
    prk = _param(r_k, C, "r_k")
    psc = _param(ln_scale, C, "ln_scale")
    pbi = _param(ln_bias, C, "ln_bias")
    if out is None:
        out = [torch.empty_like(y) for _ in range(4)] + [
            torch.empty_like(g)] + [
            torch.empty(C, dtype=torch.float32, device=dev)
            for _ in range(3)]
    P = wkv_hip._p
    _call("rwkv7m_timemix_wkv_output_backward_noalloc",
          wkv_hip._dtype_code(g), rows, H, head_size, P(y), P(r), P(k), P(v),
          P(g), P(prk), P(psc), P(pbi), float(eps), P(dout), *map(P, out),
          wkv_hip._stream(dev))
    return tuple(out)
