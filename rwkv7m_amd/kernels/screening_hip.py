"""HIP (gfx950) kernels of the state-level screening read path: ctypes
binding of the ``rwkv7m_screen_*`` entry points of librwkv7m_wkv.so
(include/rwkv7m_screening.h).

``slot_scan`` / ``slot_scan_backward``: the slot recurrence of the
read-only scan (src/rwkv7m/model/nnx_model.py:1087-1102) for every step at
once.  ``write`` / ``write_backward``: the read/write phase's recurrence
(:1040-1047, :1103-1115).  ``read`` / ``read_backward``: the per-token read
(nnx_model.py:1063-1086).  Tensors are torch device tensors; there is no
CPU fallback.
"""

from __future__ import annotations

import torch

from . import wkv_hip


def _call(fn: str, *args) -> None:
    lib = wkv_hip.load_library()
    wkv_hip._check(getattr(lib, fn)(*args), fn)


def _c(t):
    return None if t is None else t.contiguous()


def _f32(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _check(named):
    """Each (name, tensor or None, shape): the exact shape, and every given
    tensor on one GPU (the kernels take bare pointers)."""
    for name, t, shape in named:
        if t is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} has shape {tuple(t.shape)}; expected "
                             f"{tuple(shape)}")
    return wkv_hip._dev([t for _, t, _ in named if t is not None])


def _scalar(name, t):
    if t.numel() != 1:
        raise ValueError(f"{name} must hold one value, got shape "
                         f"{tuple(t.shape)}")


def _workspace(B, T, M, ds, dev):
    n = wkv_hip.load_library().rwkv7m_screen_slot_scan_workspace_floats(
        B, T, M, ds)
    if n < 0:
        raise ValueError(f"invalid slot-scan sizes B={B} T={T} M={M} ds={ds}")
    return torch.empty(max(n, 1), dtype=torch.float32, device=dev), n


def slot_scan(base, slot_term, mu, slots0):
    """base [B, T, ds] (bf16/fp32), slot_term [M, ds], mu [M], slots0
    [B, M, ds] -> (slots_seq [B, T, M, ds] in base's dtype, slots_T
    [B, M, ds] fp32, upd2 [B, T, M, ceil(ds/64)] fp32)."""
    base = _c(base)
    B, T, ds = base.shape
    M = slot_term.shape[0]
    dev = _check([("base", base, (B, T, ds)), ("slot_term", slot_term, (M, ds)),
                  ("mu", mu, (M,)), ("slots0", slots0, (B, M, ds))])
    st, mu_, s0 = _f32(slot_term), _f32(mu), _f32(slots0)
    seq = torch.empty(B, T, M, ds, dtype=base.dtype, device=dev)
    s_t = torch.empty(B, M, ds, dtype=torch.float32, device=dev)
    upd2 = torch.empty(B, T, M, (ds + 63) // 64, dtype=torch.float32,
                       device=dev)
    ws, nws = _workspace(B, T, M, ds, dev)
    P = wkv_hip._p
    _call("rwkv7m_screen_slot_scan", wkv_hip._dtype_code(base), B, T, M, ds,
          P(base), P(st), P(mu_), P(s0), P(seq), P(s_t), P(upd2), P(ws), nws,
          wkv_hip._stream(dev))
    return seq, s_t, upd2


def slot_scan_backward(base, slot_term, mu, slots_seq, d_slots_seq,
                       d_slots_T=None):
    """-> (d_pre [B, T, M, ds] fp32, d_slots0 [B, M, ds], d_mu_part
    [B, M, ds]); d base = d_pre.sum(2), d slot_term = d_pre.sum((0, 1)),
    d mu = d_mu_part.sum((0, 2))."""
    base, slots_seq = _c(base), _c(slots_seq)
    d_slots_seq = _c(d_slots_seq).to(base.dtype)
    B, T, ds = base.shape
    M = slot_term.shape[0]
    dev = _check([("base", base, (B, T, ds)), ("slot_term", slot_term, (M, ds)),
                  ("mu", mu, (M,)), ("slots_seq", slots_seq, (B, T, M, ds)),
                  ("d_slots_seq", d_slots_seq, (B, T, M, ds)),
                  ("d_slots_T", d_slots_T, (B, M, ds))])
    st, mu_ = _f32(slot_term), _f32(mu)
    dst = _f32(d_slots_T)
    d_pre = torch.empty(B, T, M, ds, dtype=torch.float32, device=dev)
    d_s0 = torch.empty(B, M, ds, dtype=torch.float32, device=dev)
    d_mu = torch.empty(B, M, ds, dtype=torch.float32, device=dev)
    ws, nws = _workspace(B, T, M, ds, dev)
    P = wkv_hip._p
    _call("rwkv7m_screen_slot_scan_backward", wkv_hip._dtype_code(base), B,
          T, M, ds, P(base), P(st), P(mu_), P(slots_seq), P(d_slots_seq),
          P(dst), P(d_pre), P(d_s0), P(d_mu), P(ws), nws,
          wkv_hip._stream(dev))
    return d_pre, d_s0, d_mu


def _read_scalars(cfg, tau):
    """(tau on the device, trim_eps, value_unit_norm, leaky, alpha, gamma,
    cap, eps).  tau stays a device tensor: no host synchronisation, so the
    call can be captured in a HIP graph."""
    leaky = bool(cfg.use_leaky_warmup)
    trim_eps = 1e-6 if leaky else float(cfg.eps)  # nnx_model.py:1071, :1075
    tau_d = tau.detach().to(torch.float32).reshape(1).contiguous()
    return (tau_d, trim_eps, int(bool(cfg.use_value_unit_norm)),
            int(leaky), float(cfg.leaky_alpha), float(cfg.leaky_gamma),
            float(cfg.tanh_norm_cap), float(cfg.eps))


def read(q, proj, tau, age_w, cfg, dv):
    """q [B, T, dk] fp32, proj [B, T, M, dk + dv], tau a device scalar
    tensor -> (u [B, T, dv] in
    proj's dtype, rel [B, T, M], z_norm [B, T], u_norm [B, T])."""
    q, proj = _f32(q), _c(proj)
    B, T, M, kv = proj.shape
    dk = kv - dv
    _scalar("tau", tau)
    dev = _check([("q", q, (B, T, dk)), ("proj", proj, (B, T, M, kv)),
                  ("age_w", age_w, (B, T, M) if age_w is not None and
                   age_w.dim() == 3 else (B, M)), ("tau", tau, tau.shape)])
    aw = _f32(age_w)
    u = torch.empty(B, T, dv, dtype=proj.dtype, device=dev)
    rel = torch.empty(B, T, M, dtype=torch.float32, device=dev)
    zn = torch.empty(B, T, dtype=torch.float32, device=dev)
    un = torch.empty(B, T, dtype=torch.float32, device=dev)
    sc = _read_scalars(cfg, tau)
    per_step = int(aw is not None and aw.dim() == 3)
    P = wkv_hip._p
    _call("rwkv7m_screen_read", wkv_hip._dtype_code(proj), B, T, M, dk, dv,
          P(q), P(proj), P(sc[0]), sc[1], P(aw), per_step, *sc[2:], P(u),
          P(rel), P(zn), P(un), wkv_hip._stream(dev))
    return u, rel, zn, un


def read_backward(q, proj, tau, age_w, cfg, dv, du, d_rel=None):
    """-> (dq [B, T, dk] fp32, d_proj like proj, d_tau [B, T], g_age
    [B, T, M]) with d age_w = g_age.sum(1)."""
    q, proj = _f32(q), _c(proj)
    du = _c(du).to(proj.dtype)
    B, T, M, kv = proj.shape
    dk = kv - dv
    _scalar("tau", tau)
    dev = _check([("q", q, (B, T, dk)), ("proj", proj, (B, T, M, kv)),
                  ("age_w", age_w, (B, T, M) if age_w is not None and
                   age_w.dim() == 3 else (B, M)), ("tau", tau, tau.shape),
                  ("du", du, (B, T, dv)), ("d_rel", d_rel, (B, T, M))])
    aw, dr = _f32(age_w), _f32(d_rel)
    dq = torch.empty(B, T, dk, dtype=torch.float32, device=dev)
    dproj = torch.empty_like(proj)
    dtau = torch.empty(B, T, dtype=torch.float32, device=dev)
    g_age = torch.empty(B, T, M, dtype=torch.float32, device=dev)
    sc = _read_scalars(cfg, tau)
    per_step = int(aw is not None and aw.dim() == 3)
    P = wkv_hip._p
    _call("rwkv7m_screen_read_backward", wkv_hip._dtype_code(proj), B, T, M,
          dk, dv, P(q), P(proj), P(sc[0]), sc[1], P(aw), per_step, *sc[2:],
          P(du), P(dr), P(dq), P(dproj), P(dtau), P(g_age),
          wkv_hip._stream(dev))
    return dq, dproj, dtau, g_age


def _write_common(base, slot_term, slot_embed, kw, q_w, tau_w, mu):
    B, T, ds = base.shape
    M, dk = slot_term.shape[0], kw.shape[-1]
    _scalar("tau_w", tau_w)
    _check([("base", base, (B, T, ds)), ("slot_term", slot_term, (M, ds)),
            ("slot_embed", slot_embed, (M, ds)), ("k_proj_w", kw, (ds, dk)),
            ("q_w", q_w, (B, T, dk)), ("tau_w", tau_w, tau_w.shape),
            ("mu", mu, (M,))])
    return (_c(base), _f32(slot_term), _f32(slot_embed), _f32(kw), _f32(q_w),
            tau_w.detach().to(torch.float32).reshape(1).contiguous(),
            _f32(mu))


def write(base, slot_term, slot_embed, kw, q_w, tau_w, mu, floor, eps,
          slots0, ages0):
    """The write-phase slot recurrence (read_write).  -> (slots_seq
    [B, T, M, ds] in base's dtype, slots32 fp32, ages_seq [B, T, M], rel_w
    [B, T, M], upd2 [B, T, M, ceil(ds/64)], slots_T [B, M, ds], ages_T
    [B, M])."""
    base, st, se, kw_, qw, tw, mu_ = _write_common(base, slot_term,
                                                   slot_embed, kw, q_w, tau_w,
                                                   mu)
    B, T, ds = base.shape
    M, dk = st.shape[0], kw_.shape[1]
    dev = _check([("base", base, (B, T, ds)), ("slots0", slots0, (B, M, ds)),
                  ("ages0", ages0, (B, M))])
    f = dict(dtype=torch.float32, device=dev)
    seq = torch.empty(B, T, M, ds, dtype=base.dtype, device=dev)
    s32 = torch.empty(B, T, M, ds, **f)
    ages_seq = torch.empty(B, T, M, **f)
    rel_w = torch.empty(B, T, M, **f)
    upd2 = torch.empty(B, T, M, (ds + 63) // 64, **f)
    s_t = torch.empty(B, M, ds, **f)
    a_t = torch.empty(B, M, **f)
    P = wkv_hip._p
    _call("rwkv7m_screen_write", wkv_hip._dtype_code(base), B, T, M, ds, dk,
          P(base), P(st), P(se), P(kw_), P(qw), P(tw), P(mu_), float(floor),
          float(eps), P(_f32(slots0)), P(_f32(ages0)), P(seq), P(s32),
          P(ages_seq), P(rel_w), P(upd2), P(s_t), P(a_t),
          wkv_hip._stream(dev))
    return seq, s32, ages_seq, rel_w, upd2, s_t, a_t


def write_backward(base, slot_term, slot_embed, kw, q_w, tau_w, mu, floor,
                   eps, slots32, d_slots_seq, d_slots_T=None, d_rel_w=None,
                   d_ages_seq=None, d_ages_T=None):
    """-> (d_pre [B, T, M, ds], d_slots0, d_ages0, d_embed_part [B, M, ds],
    d_mu_bm [B, M], d_kraw [B, T, M, dk], dq_w [B, T, M, dk], d_tau_w
    [B, T, M])."""
    base, st, se, kw_, qw, tw, mu_ = _write_common(base, slot_term,
                                                   slot_embed, kw, q_w, tau_w,
                                                   mu)
    B, T, ds = base.shape
    M, dk = st.shape[0], kw_.shape[1]
    dev = _check([("base", base, (B, T, ds)),
                  ("slots32", slots32, (B, T, M, ds)),
                  ("d_slots_seq", d_slots_seq, (B, T, M, ds)),
                  ("d_slots_T", d_slots_T, (B, M, ds)),
                  ("d_rel_w", d_rel_w, (B, T, M)),
                  ("d_ages_seq", d_ages_seq, (B, T, M)),
                  ("d_ages_T", d_ages_T, (B, M))])
    f = dict(dtype=torch.float32, device=dev)
    d_seq = _c(d_slots_seq).to(base.dtype)
    outs = [torch.empty(B, T, M, ds, **f), torch.empty(B, M, ds, **f),
            torch.empty(B, M, **f), torch.empty(B, M, ds, **f),
            torch.empty(B, M, **f), torch.empty(B, T, M, dk, **f),
            torch.empty(B, T, M, dk, **f), torch.empty(B, T, M, **f)]
    P = wkv_hip._p
    _call("rwkv7m_screen_write_backward", wkv_hip._dtype_code(base), B, T, M,
          ds, dk, P(base), P(st), P(se), P(kw_), P(qw), P(tw), P(mu_),
          float(floor), float(eps), P(_f32(slots32)), P(d_seq),
          P(_f32(d_slots_T)), P(_f32(d_rel_w)), P(_f32(d_ages_seq)),
          P(_f32(d_ages_T)), *map(P, outs), wkv_hip._stream(dev))
    return tuple(outs)
