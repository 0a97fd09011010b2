"""TEST INFRASTRUCTURE ONLY: float64 numpy oracle of the state-level screening
read path (phase ``read_screening_only``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or as
the timed CPU baseline.  No product code path imports it.

Restates ``NNXStateLevelScreening.__call__`` (src/rwkv7m/model/
nnx_model.py:999-1160) step by step, as its ``jax.lax.scan`` runs it, with
the helpers of src/rwkv7m/model/screening.py:

* ``unit_norm`` (:21-24), ``bounded_tau`` (:27-28), ``trim_square``
  (:37-39), ``tanh_norm`` (:48-52), ``update_rate_from_half_life`` (:55-58),
  ``compute_slot_delta`` (:61-88, ``tanh`` of the split projection);
* ``_compute_mu`` (nnx_model.py:1002-1013): per-bank rates gathered by
  ``bank_ids``;
* the screen LayerNorm (flax LayerNorm, epsilon 1e-6, fp32 statistics,
  variance E[x^2] - E[x]^2 clamped at 0);
* the read-only step (:1062-1112 with ``write_enabled`` false): keys and
  values of the current slots, relevance, the read, the gated residual, then
  ``slots + mu * (delta - slots)`` and the usage EMA; ages are unchanged;
* the read/write step (``phase="read_write"``, :1040-1047 and :1103-1115):
  write keys of ``slots + slot_embed``, write relevance against the write
  query, the update scaled by ``mu * max(rel_w, write_rel_floor)``, ages
  reset where ``rel_w > 1e-3``, usage fed by ``max(rel, rel_w)``;
* the statistics (:1117-1137), averaged over the steps.

Parameters are a dict of float64 arrays named as the reference's module
attributes; linear kernels are ``[in, out]`` (flax layout).  Pinning:
``tests/test_screening_oracle.py``.
"""

from __future__ import annotations

import numpy as np

PARAM_NAMES = ("ln_scale", "ln_bias", "q_proj_r", "k_proj_r", "v_proj",
               "out_proj", "gate_kernel", "gate_bias", "delta_kernel",
               "delta_bias", "tau_r_raw", "lambda_raw", "slot_embed",
               "mu_by_bank_raw")

STAT_NAMES = ("rel_read_mean", "rel_read_max", "active_slots_mean",
              "z_norm_mean", "u_norm_mean", "tau_r", "lambda_screen",
              "rel_write_mean", "rel_write_effective_mean",
              "slot_update_norm_mean", "slot_usage_ema_mean", "tau_w")


def sigmoid(x):
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def softplus(x):
    return np.logaddexp(x, 0.0)


def unit_norm(x, eps):
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps * eps)


def trim_square(sim, tau, eps):
    x = (sim - tau) / (1.0 - tau + eps)
    return np.square(np.maximum(x, 0.0))


def tanh_norm(z, cap, eps):
    n = np.sqrt((z * z).sum(-1, keepdims=True) + eps * eps)
    return cap * np.tanh(n / cap) / n * z


def layer_norm(x, scale, bias, eps=1e-6):
    mean = x.mean(-1, keepdims=True)
    var = np.maximum((x * x).mean(-1, keepdims=True) - mean * mean, 0.0)
    return (x - mean) / np.sqrt(var + eps) * scale + bias


def compute_mu(cfg, mu_by_bank_raw):
    """nnx_model.py:1002-1013."""
    mu_max = np.array([cfg["mu_short_max"], cfg["mu_mid_max"],
                       cfg["mu_long_max"]])
    legacy = mu_max * sigmoid(np.asarray(mu_by_bank_raw, np.float64))
    per_bank = []
    for i, hl in enumerate((cfg["short_half_life_tokens"],
                            cfg["mid_half_life_tokens"],
                            cfg["long_half_life_tokens"])):
        per_bank.append(legacy[i] if hl is None
                        else -np.expm1(-np.log(2.0) / hl))
    return np.stack(per_bank)[np.asarray(cfg["bank_ids"], np.int64)]


def read_forward(x, h_base, slots, ages, usage, P, cfg,
                 phase="read_screening_only"):
    """One call in ``phase`` (``read_screening_only`` or ``read_write``; the
    write path needs ``cfg["use_write_screening"]`` and the parameters
    ``q_proj_w``, ``k_proj_w``, ``tau_w_raw``).

    x, h_base: [B, T, C]; slots [B, M, d_slot]; ages, usage [B, M].
    Returns (h [B, T, C], (slots_T, ages_T, usage_T), stats dict).
    """
    eps = cfg["eps"]
    write = phase == "read_write" and cfg.get("use_write_screening", False)
    B, T, C = x.shape
    x_ln = layer_norm(x, P["ln_scale"], P["ln_bias"])
    q = unit_norm(x_ln @ P["q_proj_r"], eps)
    tau = 2.0 * sigmoid(P["tau_r_raw"]) - 1.0
    lam = softplus(P["lambda_raw"])
    mu = compute_mu(cfg, P["mu_by_bank_raw"])
    gate = sigmoid(x_ln @ P["gate_kernel"] + P["gate_bias"])
    dk = P["delta_kernel"]
    x_term = x_ln @ dk[:C]
    h_term = h_base @ dk[C:2 * C]
    slot_term = P["slot_embed"] @ dk[2 * C:]
    if write:  # nnx_model.py:1040-1047
        q_w = unit_norm(np.concatenate([x_ln, h_base], -1) @ P["q_proj_w"],
                        eps)
        tau_w = 2.0 * sigmoid(P["tau_w_raw"]) - 1.0
    hs = np.empty_like(h_base)
    acc = {n: 0.0 for n in STAT_NAMES}
    for t in range(T):
        age_w = (sigmoid((cfg["age_ref"] - ages) / (cfg["age_sigma"] + eps))
                 if cfg["use_age_mask"] else None)
        k_r = unit_norm(slots @ P["k_proj_r"], eps)
        values = slots @ P["v_proj"]
        if cfg["use_value_unit_norm"]:
            values = unit_norm(values, eps)
        sim = np.einsum("bk,bmk->bm", q[:, t], k_r)
        if cfg["use_leaky_warmup"]:
            hard = trim_square(sim, tau, 1e-6)
            soft = sigmoid(cfg["leaky_gamma"] * (sim - tau))
            rel = (1.0 - cfg["leaky_alpha"]) * hard + cfg["leaky_alpha"] * soft
        else:
            rel = trim_square(sim, tau, eps)
        if age_w is not None:
            rel = rel * age_w
        z = np.einsum("bm,bmv->bv", rel, values)
        u = tanh_norm(z, cfg["tanh_norm_cap"], eps)
        read = u @ P["out_proj"]
        hs[:, t] = h_base[:, t] + lam * gate[:, t] * read
        delta = np.tanh(x_term[:, t, None, :] + h_term[:, t, None, :]
                        + slot_term[None] + P["delta_bias"])
        if write:  # nnx_model.py:1103-1115
            k_w = unit_norm((slots + P["slot_embed"][None]) @ P["k_proj_w"],
                            eps)
            rel_w = trim_square(np.einsum("bk,bmk->bm", q_w[:, t], k_w),
                                tau_w, eps)
            strength = mu[None, :] * np.maximum(rel_w, cfg["write_rel_floor"])
            new_slots = slots + strength[:, :, None] * (delta - slots)
            ages = np.where(rel_w > 1e-3, 0.0, ages + 1.0)
            activity = np.maximum(rel, rel_w)
            acc["rel_write_mean"] += rel_w.mean()
            acc["rel_write_effective_mean"] += np.maximum(
                rel_w, cfg["write_rel_floor"]).mean()
            acc["tau_w"] += tau_w
        else:
            new_slots = slots + mu[None, :, None] * (delta - slots)
            activity = rel
        upd = new_slots - slots
        usage = cfg["usage_ema_decay"] * usage + (
            1.0 - cfg["usage_ema_decay"]) * activity
        acc["rel_read_mean"] += rel.mean()
        acc["rel_read_max"] += rel.max()
        acc["active_slots_mean"] += (rel > 1e-3).sum(-1).mean()
        acc["z_norm_mean"] += np.linalg.norm(z, axis=-1).mean()
        acc["u_norm_mean"] += np.linalg.norm(u, axis=-1).mean()
        acc["tau_r"] += tau
        acc["lambda_screen"] += lam
        acc["slot_update_norm_mean"] += np.linalg.norm(upd, axis=-1).mean()
        acc["slot_usage_ema_mean"] += usage.mean()
        slots = new_slots
    stats = {n: float(v) / T for n, v in acc.items()}
    return hs, (slots, ages, usage), stats


def read_forward_torch(x, h_base, slots, ages, usage, P, cfg,
                       phase="read_screening_only"):
    """The same step-by-step scan with torch float64 ops, for autograd (the
    gradient oracle): arguments are float64 torch tensors, P a dict of
    them.  Returns (h, slots_T, usage_T)."""
    import torch

    eps = cfg["eps"]
    write = phase == "read_write" and cfg.get("use_write_screening", False)
    B, T, C = x.shape

    def un(v):
        return v / torch.sqrt((v * v).sum(-1, keepdim=True) + eps * eps)

    def trim(sim, tau, e):
        return torch.clamp((sim - tau) / (1.0 - tau + e), min=0.0) ** 2

    mean = x.mean(-1, keepdim=True)
    var = torch.clamp((x * x).mean(-1, keepdim=True) - mean * mean, min=0.0)
    x_ln = (x - mean) / torch.sqrt(var + 1e-6) * P["ln_scale"] + P["ln_bias"]
    q = un(x_ln @ P["q_proj_r"])
    tau = 2.0 * torch.sigmoid(P["tau_r_raw"]) - 1.0
    lam = torch.nn.functional.softplus(P["lambda_raw"])
    mu_max = torch.tensor([cfg["mu_short_max"], cfg["mu_mid_max"],
                           cfg["mu_long_max"]], dtype=x.dtype)
    legacy = mu_max * torch.sigmoid(P["mu_by_bank_raw"])
    banks = []
    for i, hl in enumerate((cfg["short_half_life_tokens"],
                            cfg["mid_half_life_tokens"],
                            cfg["long_half_life_tokens"])):
        banks.append(legacy[i] if hl is None else torch.tensor(
            -np.expm1(-np.log(2.0) / hl), dtype=x.dtype))
    mu = torch.stack(banks)[torch.tensor(cfg["bank_ids"])]
    gate = torch.sigmoid(x_ln @ P["gate_kernel"] + P["gate_bias"])
    dk = P["delta_kernel"]
    x_term = x_ln @ dk[:C]
    h_term = h_base @ dk[C:2 * C]
    slot_term = P["slot_embed"] @ dk[2 * C:]
    if write:
        q_w = un(torch.cat([x_ln, h_base], -1) @ P["q_proj_w"])
        tau_w = 2.0 * torch.sigmoid(P["tau_w_raw"]) - 1.0
    hs = []
    for t in range(T):
        age_w = (torch.sigmoid((cfg["age_ref"] - ages)
                               / (cfg["age_sigma"] + eps))
                 if cfg["use_age_mask"] else None)
        k_r = un(slots @ P["k_proj_r"])
        values = slots @ P["v_proj"]
        if cfg["use_value_unit_norm"]:
            values = un(values)
        sim = torch.einsum("bk,bmk->bm", q[:, t], k_r)
        if cfg["use_leaky_warmup"]:
            rel = ((1.0 - cfg["leaky_alpha"]) * trim(sim, tau, 1e-6)
                   + cfg["leaky_alpha"]
                   * torch.sigmoid(cfg["leaky_gamma"] * (sim - tau)))
        else:
            rel = trim(sim, tau, eps)
        if age_w is not None:
            rel = rel * age_w
        z = torch.einsum("bm,bmv->bv", rel, values)
        n = torch.sqrt((z * z).sum(-1, keepdim=True) + eps * eps)
        cap = cfg["tanh_norm_cap"]
        u = cap * torch.tanh(n / cap) / n * z
        hs.append(h_base[:, t] + lam * gate[:, t] * (u @ P["out_proj"]))
        delta = torch.tanh(x_term[:, t, None, :] + h_term[:, t, None, :]
                           + slot_term[None] + P["delta_bias"])
        if write:
            k_w = un((slots + P["slot_embed"][None]) @ P["k_proj_w"])
            rel_w = trim(torch.einsum("bk,bmk->bm", q_w[:, t], k_w), tau_w,
                         eps)
            strength = mu[None, :] * torch.clamp(
                rel_w, min=cfg["write_rel_floor"])
            slots = slots + strength[:, :, None] * (delta - slots)
            ages = torch.where(rel_w > 1e-3, torch.zeros_like(ages),
                               ages + 1.0)
            activity = torch.maximum(rel, rel_w)
        else:
            slots = slots + mu[None, :, None] * (delta - slots)
            activity = rel
        usage = cfg["usage_ema_decay"] * usage + (
            1.0 - cfg["usage_ema_decay"]) * activity
    return torch.stack(hs, 1), slots, usage


# Tolerances of scalar_grad_error.  fp32: 1e-4 of the gradient's own
# magnitude, unless the sum cancelled by more than 1000x (|grad| / sum|terms|
# below HEAVY_CANCELLATION), where fp32 rounding of the terms alone (6e-8
# each) can exceed 1e-4 of the result: then 1e-6 of the terms' sum (about 16
# fp32 roundings).  bf16: 4e-3 of the terms' sum (two bf16 roundings, 2^-8).
SCALAR_TOL_FP32 = 1e-4
SCALAR_TOL_FP32_TERMS = 1e-6
HEAVY_CANCELLATION = 1e-3
SCALAR_TOL_BF16 = 4e-3


def scalar_grad_error(got, want, term_scale, fp32):
    """Error of a scalar parameter's gradient ``got`` against ``want``, whose
    terms (one per output element: cotangent times derivative) have
    magnitudes summing to ``term_scale``.

    Returns ``(error, ratio, basis, tol)`` with ``ratio = |want| /
    term_scale``, the share of the terms that survives their cancellation.
    fp32: relative to ``|want|`` (tol 1e-4) unless ``ratio <
    HEAVY_CANCELLATION``, then relative to ``term_scale`` (tol 1e-6).  bf16:
    relative to ``term_scale`` (tol 4e-3).  Relative to ``term_scale``, a
    relative error ``e`` of the gradient reads as ``e * ratio`` and a missing
    group of terms as its share of ``term_scale``."""
    ratio = abs(want) / term_scale if term_scale > 0 else 0.0
    terms = abs(got - want) / term_scale if term_scale > 0 else abs(got - want)
    if fp32 and ratio >= HEAVY_CANCELLATION:
        return abs(got - want) / abs(want), ratio, "own magnitude", \
            SCALAR_TOL_FP32
    if fp32:
        return terms, ratio, "terms", SCALAR_TOL_FP32_TERMS
    return terms, ratio, "terms", SCALAR_TOL_BF16


def default_config(**overrides):
    """The reference's ScreeningConfig defaults (screening.py:92-121) as a
    dict, with overrides."""
    cfg = dict(d_model=512, d_slot=256, d_k=64, d_v=128, n_slots=16,
               bank_ids=(), tau_init=0.0, tanh_norm_cap=1.0,
               lambda_screen_init=0.01, eps=1e-6, use_value_unit_norm=True,
               use_age_mask=False, use_leaky_warmup=False, leaky_alpha=0.0,
               leaky_gamma=8.0, mu_short_max=0.05, mu_mid_max=0.02,
               mu_long_max=0.005, short_half_life_tokens=None,
               mid_half_life_tokens=None, long_half_life_tokens=None,
               usage_ema_decay=0.99, age_ref=32.0, age_sigma=8.0,
               use_write_screening=False, write_rel_floor=1e-3)
    cfg.update(overrides)
    return cfg
