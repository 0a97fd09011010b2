"""State-level screening read path on MI355X.

A torch module with the parameters and call signature of the reference's
``NNXStateLevelScreening`` (src/rwkv7m/model/nnx_model.py:885-1160) for the
phase the training loop runs, ``read_screening_only``
(train/train_loop.py:82, train/train_step.py:20).

The reference scans the sequence one token at a time, projecting every slot
to keys and values at every step.  With writes disabled the slot update
never reads the slots' keys or values, so the call reorganises into
whole-sequence work:

1. the screen LayerNorm, the query, gate and delta projections of every
   token (library GEMMs);
2. the slot recurrence ``S_{t+1} = S_t + mu (tanh(base_t + slot_term) -
   S_t)`` for all steps (HIP kernel, ``rwkv7m_screen_slot_scan``);
3. keys and values of every step's slots (one library GEMM);
4. the per-token read -- unit norms, similarity, trim-square relevance with
   the age weight, the value mix, ``tanh_norm`` (HIP kernel,
   ``rwkv7m_screen_read``);
5. the output projection and the gated residual (GEMM, elementwise).

Steps 2 and 4 have HIP backward kernels; the rest is differentiated by
torch autograd.  The read/write phase (``read_write`` with
``use_write_screening``) replaces step 2 with the write recurrence (HIP
kernels ``rwkv7m_screen_write`` and its backward), whose update strength
depends on the slots' own write keys, and feeds the read per-step ages.
Arithmetic follows the reference's dtypes: projections in the
compute dtype, statistics, norms, the slots and the usage EMA in fp32.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple

import torch
import torch.nn.functional as F

from .kernels import screening_hip

_PHASE_ALIASES = {"read_only": "read_screening_only"}
_VALID_PHASES = {"read_screening_only", "read_write"}


def normalize_phase(phase: str) -> str:
    """src/rwkv7m/model/screening.py:11-18."""
    phase = _PHASE_ALIASES.get(phase, phase)
    if phase not in _VALID_PHASES:
        raise ValueError(
            f"Unknown phase {phase!r}. Expected one of "
            f"{sorted(_VALID_PHASES)} or compatibility alias 'read_only'.")
    return phase


@dataclass
class ScreeningConfig:
    """Fields and defaults of the reference's ScreeningConfig
    (src/rwkv7m/model/screening.py:91-144)."""

    d_model: int = 512
    d_slot: int = 256
    d_k: int = 64
    d_v: int = 128
    n_slots: int = 16
    screened_layers: tuple = ()
    bank_ids: tuple = ()
    tau_init: float = 0.0
    tanh_norm_cap: float = 1.0
    lambda_screen_init: float = 0.01
    eps: float = 1e-6
    use_value_unit_norm: bool = True
    use_age_mask: bool = False
    use_bank_bias: bool = False
    use_write_screening: bool = False
    write_rel_floor: float = 1e-3
    use_leaky_warmup: bool = False
    leaky_alpha: float = 0.0
    leaky_gamma: float = 8.0
    mu_short_max: float = 0.05
    mu_mid_max: float = 0.02
    mu_long_max: float = 0.005
    short_half_life_tokens: float | None = None
    mid_half_life_tokens: float | None = None
    long_half_life_tokens: float | None = None
    usage_ema_decay: float = 0.99
    age_ref: float = 32.0
    age_sigma: float = 8.0

    def __post_init__(self):
        self.screened_layers = tuple(self.screened_layers)
        self.bank_ids = tuple(self.bank_ids)
        if self.bank_ids and len(self.bank_ids) != self.n_slots:
            raise ValueError("bank_ids must have length n_slots when provided")
        if [b for b in self.bank_ids if b not in (0, 1, 2)]:
            raise ValueError("bank_ids values must be only 0, 1, or 2")
        if self.write_rel_floor < 0.0:
            raise ValueError("write_rel_floor must be non-negative")
        for hl in (self.short_half_life_tokens, self.mid_half_life_tokens,
                   self.long_half_life_tokens):
            if hl is not None and hl <= 0.0:
                raise ValueError(
                    "memory half-life values must be positive when provided")
        if not 0.0 <= self.usage_ema_decay < 1.0:
            raise ValueError("usage_ema_decay must be in [0, 1)")


class ScreenState(NamedTuple):
    """LayerScreenState (src/rwkv7m/model/state.py:13-17)."""

    slots: torch.Tensor      # [B, M, d_slot] fp32
    ages: torch.Tensor       # [B, M]
    usage_ema: torch.Tensor  # [B, M]


def init_screen_state(batch_size: int, config: ScreeningConfig,
                      device=None) -> ScreenState:
    """state.py:24-34 for one layer: zeros."""
    z = dict(dtype=torch.float32, device=device)
    return ScreenState(
        torch.zeros(batch_size, config.n_slots, config.d_slot, **z),
        torch.zeros(batch_size, config.n_slots, **z),
        torch.zeros(batch_size, config.n_slots, **z))


def _theta_from_tau(tau: float) -> float:
    p = min(max((tau + 1.0) / 2.0, 1e-4), 1.0 - 1e-4)
    return math.log(p) - math.log1p(-p)


class _SlotScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, base, slot_term, mu, slots0):
        seq, s_t, upd2 = screening_hip.slot_scan(base, slot_term, mu, slots0)
        ctx.save_for_backward(base, slot_term, mu, seq)
        ctx.mark_non_differentiable(upd2)
        return seq, s_t, upd2

    @staticmethod
    def backward(ctx, d_seq, d_s_t, _d_upd2):
        base, slot_term, mu, seq = ctx.saved_tensors
        if d_seq is None:
            d_seq = torch.zeros_like(seq)
        d_pre, d_s0, d_mu = screening_hip.slot_scan_backward(
            base, slot_term, mu, seq, d_seq, d_s_t)
        return (d_pre.sum(2).to(base.dtype),
                d_pre.sum((0, 1)).to(slot_term.dtype),
                d_mu.sum((0, 2)).to(mu.dtype), d_s0)


class _ScreenRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, proj, tau, age_w, cfg, dv):
        u, rel, zn, un = screening_hip.read(q, proj, tau, age_w, cfg, dv)
        ctx.save_for_backward(q, proj, tau, age_w)
        ctx.cfg, ctx.dv = cfg, dv
        ctx.mark_non_differentiable(zn, un)
        return u, rel, zn, un

    @staticmethod
    def backward(ctx, du, d_rel, _dzn, _dun):
        q, proj, tau, age_w = ctx.saved_tensors
        if du is None:
            du = torch.zeros(*proj.shape[:2], ctx.dv, dtype=proj.dtype,
                             device=proj.device)
        dq, dproj, dtau, g_age = screening_hip.read_backward(
            q, proj, tau, age_w, ctx.cfg, ctx.dv, du, d_rel)
        d_age = None
        if age_w is not None:  # [B, M] (summed over steps) or [B, T, M]
            d_age = g_age.sum(1) if age_w.dim() == 2 else g_age
        return (dq, dproj, dtau.sum().reshape(tau.shape).to(tau.dtype),
                d_age, None, None)


class _SlotProjection(torch.autograd.Function):
    """keys and values of every step's slots: seq [B, T, M, ds] @ kv
    [ds, dk + dv].  The weight gradient is a reduction over B*T*M rows; it
    runs as one batched product per batch row, summed in fp32, instead of a
    single long-K GEMM."""

    @staticmethod
    def forward(ctx, seq, kv):
        ctx.save_for_backward(seq, kv)
        return seq @ kv

    @staticmethod
    def backward(ctx, g):
        seq, kv = ctx.saved_tensors
        g = g.contiguous()
        d_seq = g @ kv.t().contiguous()
        B, ds = seq.shape[0], seq.shape[-1]
        part = torch.bmm(seq.reshape(B, -1, ds).transpose(1, 2).contiguous(),
                         g.reshape(B, -1, g.shape[-1]))
        return d_seq, part.float().sum(0).to(kv.dtype)


class _WriteScan(torch.autograd.Function):
    """The read/write phase's slot recurrence (HIP kernels
    rwkv7m_screen_write / _backward)."""

    @staticmethod
    def forward(ctx, base, slot_term, slot_embed, kw, q_w, tau_w, mu,
                slots0, ages0, floor, eps):
        seq, s32, ages_seq, rel_w, upd2, s_t, a_t = screening_hip.write(
            base, slot_term, slot_embed, kw, q_w, tau_w, mu, floor, eps,
            slots0, ages0)
        ctx.save_for_backward(base, slot_term, slot_embed, kw, q_w, tau_w,
                              mu, s32)
        ctx.floor, ctx.eps = floor, eps
        ctx.mark_non_differentiable(upd2)
        return seq, ages_seq, rel_w, upd2, s_t, a_t

    @staticmethod
    def backward(ctx, d_seq, d_ages_seq, d_rel_w, _d_upd2, d_s_t, d_a_t):
        base, slot_term, slot_embed, kw, q_w, tau_w, mu, s32 = \
            ctx.saved_tensors
        if d_seq is None:
            d_seq = torch.zeros(s32.shape, dtype=base.dtype,
                                device=base.device)
        (d_pre, d_s0, d_a0, d_emb, d_mu, d_kraw, dq_w,
         d_tau) = screening_hip.write_backward(
            base, slot_term, slot_embed, kw, q_w, tau_w, mu, ctx.floor,
            ctx.eps, s32, d_seq, d_s_t, d_rel_w, d_ages_seq, d_a_t)
        B, T, M, ds = s32.shape
        skey = (s32 + slot_embed.float()[None, None]).to(base.dtype).float()
        d_kw = torch.bmm(skey.reshape(B, -1, ds).transpose(1, 2).contiguous(),
                         d_kraw.reshape(B, -1, kw.shape[1])).sum(0)
        return (d_pre.sum(2).to(base.dtype),
                d_pre.sum((0, 1)).to(slot_term.dtype),
                d_emb.sum(0).to(slot_embed.dtype), d_kw.to(kw.dtype),
                dq_w.sum(2), d_tau.sum().reshape(tau_w.shape).to(tau_w.dtype),
                d_mu.sum(0).to(mu.dtype), d_s0, d_a0, None, None)


def _ema_time_mean(r_bar: torch.Tensor, u0: torch.Tensor,
                   d: float) -> torch.Tensor:
    """Mean over t = 0..T-1 of u_t = d u_{t-1} + (1 - d) r_t (u_{-1} = u0),
    in closed form: (u0 d (1 - d^T) / (1 - d) + sum_t r_t (1 - d^(T-t))) / T
    (u0 T in place of the first term when d = 1)."""
    T = r_bar.shape[0]
    t = torch.arange(T, device=r_bar.device, dtype=r_bar.dtype)
    head = u0 * (T if d == 1.0 else d * (1.0 - d ** T) / (1.0 - d))
    return (head + (r_bar * (1.0 - d ** (T - t))).sum()) / T


class StateLevelScreening(torch.nn.Module):
    """NNXStateLevelScreening's parameters (nnx_model.py:885-999, linear
    kernels in the flax ``[in, out]`` layout) and its read-only call."""

    def __init__(self, config: ScreeningConfig, *,
                 compute_dtype=torch.float32,
                 param_dtype=torch.float32, device=None, seed: int = 0):
        super().__init__()
        self.config = config
        self.compute_dtype = compute_dtype
        C, ds, dk, dv, M = (config.d_model, config.d_slot, config.d_k,
                            config.d_v, config.n_slots)
        g = torch.Generator().manual_seed(seed)
        kw = dict(dtype=param_dtype, device=device)

        def lecun(fan_in, fan_out):  # flax's default linear initialiser
            w = torch.randn(fan_in, fan_out, generator=g) / math.sqrt(fan_in)
            return torch.nn.Parameter(w.to(**kw))

        def const(shape, v):
            return torch.nn.Parameter(torch.full(shape, float(v), **kw))

        self.screen_ln_scale = const((C,), 1.0)
        self.screen_ln_bias = const((C,), 0.0)
        self.q_proj_r = lecun(C, dk)
        self.k_proj_r = lecun(ds, dk)
        self.v_proj = lecun(ds, dv)
        self.out_proj = lecun(dv, C)
        self.gate_kernel = lecun(C, C)
        self.gate_bias = const((C,), 0.0)
        self.delta_kernel = lecun(2 * C + ds, ds)
        self.delta_bias = const((ds,), 0.0)
        self.tau_r_raw = const((), _theta_from_tau(config.tau_init))
        self.lambda_raw = const(
            (), math.log(math.expm1(config.lambda_screen_init)))
        self.slot_embed = torch.nn.Parameter(
            (0.02 * torch.randn(M, ds, generator=g)).to(**kw))
        self.mu_by_bank_raw = const((3,), 0.0)
        if config.use_write_screening:  # nnx_model.py:977-1000
            self.q_proj_w = lecun(2 * C, dk)
            self.k_proj_w = lecun(ds, dk)
            self.tau_w_raw = const((), _theta_from_tau(config.tau_init))
        fixed = [None if hl is None else -math.expm1(-math.log(2.0) / hl)
                 for hl in (config.short_half_life_tokens,
                            config.mid_half_life_tokens,
                            config.long_half_life_tokens)]
        self.register_buffer("_mu_max", torch.tensor(
            [config.mu_short_max, config.mu_mid_max, config.mu_long_max],
            dtype=torch.float32, device=device), persistent=False)
        self.register_buffer("_mu_fixed", torch.tensor(
            [0.0 if f is None else f for f in fixed], dtype=torch.float32,
            device=device), persistent=False)
        self.register_buffer("_mu_fixed_mask", torch.tensor(
            [f is not None for f in fixed], device=device), persistent=False)
        self.register_buffer("_bank_ids", torch.tensor(
            config.bank_ids, dtype=torch.long, device=device),
            persistent=False)

    def compute_mu(self) -> torch.Tensor:
        """nnx_model.py:1002-1013: per-bank rates (mu_max * sigmoid(raw), or
        the half-life rate where one is set) gathered by bank_ids.  Built
        from device buffers only, so the call can be captured in a graph."""
        if self._bank_ids.numel() != self.config.n_slots:
            raise ValueError("bank_ids must have length n_slots")
        legacy = self._mu_max * torch.sigmoid(self.mu_by_bank_raw.float())
        per_bank = torch.where(self._mu_fixed_mask, self._mu_fixed, legacy)
        return per_bank[self._bank_ids]

    def forward(self, x_seq, h_base_seq, state: ScreenState, *,
                phase: str = "read_screening_only", deterministic=True):
        """(h_seq [B, T, C], new ScreenState, stats) as
        NNXStateLevelScreening.__call__ (nnx_model.py:1015-1160)."""
        del deterministic
        cfg = self.config
        phase = normalize_phase(phase)
        write = phase == "read_write" and cfg.use_write_screening
        if write and not hasattr(self, "k_proj_w"):
            raise ValueError("the read_write phase needs the write "
                             "parameters: build the module with "
                             "use_write_screening=True")
        eps = cfg.eps
        B, T, C = x_seq.shape
        cd = self.compute_dtype or x_seq.dtype
        x_ln = F.layer_norm(x_seq.float(), (C,), self.screen_ln_scale.float(),
                            self.screen_ln_bias.float(), eps=1e-6).to(cd)
        q = (x_ln @ self.q_proj_r.to(cd)).float()
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + eps * eps)
        tau = 2.0 * torch.sigmoid(self.tau_r_raw.float()) - 1.0
        lam = F.softplus(self.lambda_raw.float())
        mu = self.compute_mu()
        gate = torch.sigmoid(
            (x_ln @ self.gate_kernel.to(cd) + self.gate_bias.to(cd)).float())
        dker = self.delta_kernel.to(cd)
        base = (x_ln @ dker[:C] + h_base_seq.to(cd) @ dker[C:2 * C]
                + self.delta_bias.to(cd))
        slot_term = (self.slot_embed.to(cd) @ dker[2 * C:]).float()
        if write:
            # nnx_model.py:1040-1047: the write query and threshold
            q_w = torch.cat([x_ln, h_base_seq.float().to(cd)], -1) @ \
                self.q_proj_w.to(cd)
            q_w = q_w.float()
            q_w = q_w / torch.sqrt((q_w * q_w).sum(-1, keepdim=True)
                                   + eps * eps)
            tau_w = 2.0 * torch.sigmoid(self.tau_w_raw.float()) - 1.0
            kw = self.k_proj_w.to(cd)
            seq, ages_seq, rel_w, upd2, slots_t, ages_t = _WriteScan.apply(
                base, slot_term, self.slot_embed.float(), kw, q_w, tau_w, mu,
                state.slots.float(), state.ages.float(),
                float(cfg.write_rel_floor), float(eps))
            ages_for_read = ages_seq
        else:
            seq, slots_t, upd2 = _SlotScan.apply(base, slot_term, mu,
                                                 state.slots.float())
            rel_w, ages_t, ages_for_read = None, state.ages, state.ages
        age_w = (torch.sigmoid((cfg.age_ref - ages_for_read.float())
                               / (cfg.age_sigma + eps))
                 if cfg.use_age_mask else None)
        kv = torch.cat([self.k_proj_r, self.v_proj], dim=1).to(cd)
        proj = _SlotProjection.apply(seq, kv)
        u, rel, zn, un = _ScreenRead.apply(q, proj, tau, age_w, cfg,
                                           cfg.d_v)
        read = (u @ self.out_proj.to(cd)).to(h_base_seq.dtype)
        h = (h_base_seq.float() + lam * gate * read.float()).to(
            h_base_seq.dtype)
        d = float(cfg.usage_ema_decay)
        activity = rel if rel_w is None else torch.maximum(rel, rel_w)
        w = (1.0 - d) * d ** torch.arange(T - 1, -1, -1, device=rel.device,
                                          dtype=torch.float32)
        usage_t = (d ** T) * state.usage_ema.float() + torch.einsum(
            "btm,t->bm", activity, w)
        new_state = ScreenState(slots_t.to(state.slots.dtype),
                                ages_t.to(state.ages.dtype),
                                usage_t.to(state.usage_ema.dtype))
        with torch.no_grad():
            r = rel.detach()
            zero = torch.zeros((), device=r.device)
            act = activity.detach()
            u_mean = _ema_time_mean(act.mean((0, 2)).double(),
                                    state.usage_ema.double().mean(), d)
            stats = {
                "rel_read_mean": r.mean(),
                "rel_read_max": r.amax(dim=(0, 2)).mean(),
                "active_slots_mean": (r > 1e-3).sum(-1).float().mean(),
                "z_norm_mean": zn.mean(),
                "u_norm_mean": un.mean(),
                "tau_r": tau.detach(),
                "lambda_screen": lam.detach(),
                "rel_write_mean": zero if rel_w is None else rel_w.mean(),
                "rel_write_effective_mean": (
                    zero if rel_w is None else torch.clamp(
                        rel_w, min=cfg.write_rel_floor).mean()),
                "slot_update_norm_mean": upd2.sum(-1).sqrt().mean(),
                "slot_usage_ema_mean": u_mean.float(),
                "tau_w": zero if rel_w is None else tau_w.detach(),
            }
        return h, new_state, stats


__all__ = ["ScreenState", "ScreeningConfig", "StateLevelScreening",
           "init_screen_state", "normalize_phase"]
