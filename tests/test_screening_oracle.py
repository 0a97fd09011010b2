"""Pins for the screening read-path oracle (CPU only).

``oracle/screening_oracle.py`` restates NNXStateLevelScreening's read-only
scan (src/rwkv7m/model/nnx_model.py:999-1160) twice: numpy (forward and
statistics) and torch float64 (for autograd, the gradient oracle).  Pins:

* the two restatements agree on every option (age mask, leaky warm-up,
  value normalisation off, half-life rates);
* library routines: the LayerNorm against torch.nn.functional.layer_norm,
  unit_norm against F.normalize, tanh_norm's limits (u ~ z for small z,
  |u| -> cap for large z);
* closed forms: the final slots equal (1-mu)^T S0 + sum_t mu (1-mu)^{T-1-t}
  delta_t, the final usage the same EMA of the relevances; zero slots read
  nothing at the first step (tau = 0), so h_0 = h_base_0;
* the torch restatement's autograd against central finite differences of
  the numpy forward, for every input and parameter;
* hand-built cases (two channels, three unit slots) whose relevances,
  read, gated residual, final slots, usage, ages and twelve statistics
  have short closed forms, for every option and the write phase;
* planted mistakes fail those pins: the read taken after the slot update
  (zero slots then read something), a wrong per-slot rate in the numpy
  restatement (the torch restatement, which derives the rates on its own,
  disagrees), and tanh_norm, the trim's square, softplus, the gate's sigmoid
  or the LayerNorm dropped (the hand-built case disagrees).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import screening_oracle as so

OPTIONS = [dict(), dict(use_age_mask=True), dict(use_leaky_warmup=True,
                                                 leaky_alpha=0.3),
           dict(use_value_unit_norm=False),
           dict(short_half_life_tokens=4.0, long_half_life_tokens=50.0)]


def _case(B=2, T=5, C=8, ds=6, dk=4, dv=5, M=3, seed=0, **opt):
    rng = np.random.default_rng(seed + 1000)
    wparams = {"q_proj_w": rng.normal(size=(2 * C, dk)) / np.sqrt(2 * C),
               "k_proj_w": rng.normal(size=(ds, dk)) / np.sqrt(ds),
               "tau_w_raw": np.array(-0.8)}
    rng = np.random.default_rng(seed)
    cfg = so.default_config(d_model=C, d_slot=ds, d_k=dk, d_v=dv, n_slots=M,
                            bank_ids=tuple(int(i) for i in
                                           rng.integers(0, 3, M)), **opt)
    P = {"ln_scale": 1.0 + 0.1 * rng.normal(size=C),
         "ln_bias": 0.1 * rng.normal(size=C),
         "q_proj_r": rng.normal(size=(C, dk)) / np.sqrt(C),
         "k_proj_r": rng.normal(size=(ds, dk)) / np.sqrt(ds),
         "v_proj": rng.normal(size=(ds, dv)) / np.sqrt(ds),
         "out_proj": rng.normal(size=(dv, C)) / np.sqrt(dv),
         "gate_kernel": rng.normal(size=(C, C)) / np.sqrt(C),
         "gate_bias": 0.1 * rng.normal(size=C),
         "delta_kernel": rng.normal(size=(2 * C + ds, ds)) / np.sqrt(C),
         "delta_bias": 0.1 * rng.normal(size=ds),
         "tau_r_raw": np.array(-0.4), "lambda_raw": np.array(0.3),
         "slot_embed": 0.5 * rng.normal(size=(M, ds)),
         "mu_by_bank_raw": rng.normal(size=3)}
    if opt.get("use_write_screening"):
        P.update(wparams)
    x = rng.normal(size=(B, T, C))
    h = rng.normal(size=(B, T, C))
    slots = 0.5 * rng.normal(size=(B, M, ds))
    ages = rng.uniform(0, 60, size=(B, M))
    usage = rng.uniform(0, 0.2, size=(B, M))
    return x, h, slots, ages, usage, P, cfg


def _t(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=grad)


@pytest.mark.parametrize("opt", OPTIONS, ids=str)
def test_numpy_and_torch_restatements_agree(opt):
    x, h, slots, ages, usage, P, cfg = _case(seed=1, **opt)
    hn, (sn, _, un), stats = so.read_forward(x, h, slots, ages, usage, P,
                                             cfg)
    ht, st, ut = so.read_forward_torch(
        _t(x), _t(h), _t(slots), _t(ages), _t(usage),
        {k: _t(v) for k, v in P.items()}, cfg)
    np.testing.assert_allclose(hn, ht.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(sn, st.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(un, ut.numpy(), rtol=1e-12, atol=1e-13)
    assert set(stats) == set(so.STAT_NAMES)
    assert 0.0 <= stats["rel_read_mean"] <= stats["rel_read_max"]
    assert stats["rel_write_mean"] == 0.0 and stats["tau_w"] == 0.0


def test_library_routines_and_limits():
    rng = np.random.default_rng(2)
    x = rng.normal(size=(4, 7)) * 3 + 1
    sc, bi = rng.normal(size=7), rng.normal(size=7)
    np.testing.assert_allclose(
        so.layer_norm(x, sc, bi),
        F.layer_norm(_t(x), (7,), _t(sc), _t(bi), eps=1e-6).numpy(),
        rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(so.unit_norm(x, 0.0),
                               F.normalize(_t(x), dim=-1).numpy(),
                               rtol=1e-14)
    z = rng.normal(size=(3, 5))
    np.testing.assert_allclose(so.tanh_norm(1e-6 * z, 1.0, 0.0), 1e-6 * z,
                               rtol=1e-9)
    big = so.tanh_norm(1e3 * z, 2.0, 1e-6)
    np.testing.assert_allclose(np.linalg.norm(big, axis=-1), 2.0, rtol=1e-12)
    sim = np.linspace(-1, 1, 11)
    r = so.trim_square(sim, 0.2, 1e-6)
    assert np.all(r[sim <= 0.2] == 0.0) and np.all(np.diff(r) >= 0.0)


def test_closed_forms_of_the_recurrences():
    x, h, slots, ages, usage, P, cfg = _case(seed=3, T=7)
    _, (s_t, ages_t, u_t), _ = so.read_forward(x, h, slots, ages, usage, P,
                                               cfg)
    C = x.shape[-1]
    x_ln = so.layer_norm(x, P["ln_scale"], P["ln_bias"])
    dker = P["delta_kernel"]
    delta = np.tanh((x_ln @ dker[:C] + h @ dker[C:2 * C])[:, :, None, :]
                    + (P["slot_embed"] @ dker[2 * C:])[None, None]
                    + P["delta_bias"])
    mu = so.compute_mu(cfg, P["mu_by_bank_raw"])[None, :, None]
    T = x.shape[1]
    want = (1 - mu) ** T * slots + sum(
        mu * (1 - mu) ** (T - 1 - t) * delta[:, t] for t in range(T))
    np.testing.assert_allclose(s_t, want, rtol=1e-12, atol=1e-13)
    assert ages_t is ages
    # usage: the same EMA, decay 0.99, of relevances in [0, 1] from >= 0
    assert np.all(u_t >= 0.99 ** T * usage - 1e-15)
    # zero slots and tau = 0 read nothing at the first step
    P0 = dict(P, tau_r_raw=np.array(0.0))
    h0, _, _ = so.read_forward(x, h, np.zeros_like(slots), ages, usage, P0,
                               cfg)
    np.testing.assert_array_equal(h0[:, 0], h[:, 0])
    assert np.max(np.abs(h0[:, 1:] - h[:, 1:])) > 1e-6


def test_torch_autograd_matches_finite_differences():
    x, h, slots, ages, usage, P, cfg = _case(B=1, T=3, C=4, ds=3, dk=3,
                                             dv=3, M=2, seed=4,
                                             use_age_mask=True)
    rng = np.random.default_rng(40)
    cot_h = rng.normal(size=x.shape)
    cot_s = rng.normal(size=slots.shape)
    cot_u = rng.normal(size=usage.shape)
    names = ["x", "h", "slots", "ages", "usage"] + sorted(P)
    arrays = dict(x=x, h=h, slots=slots, ages=ages, usage=usage, **P)
    tin = {k: _t(v, True) for k, v in arrays.items()}
    ht, st, ut = so.read_forward_torch(
        tin["x"], tin["h"], tin["slots"], tin["ages"], tin["usage"],
        {k: tin[k] for k in P}, cfg)
    loss = ((ht * _t(cot_h)).sum() + (st * _t(cot_s)).sum()
            + (ut * _t(cot_u)).sum())
    grads = dict(zip(names, torch.autograd.grad(loss, [tin[n]
                                                       for n in names])))

    def objective(a):
        hh, (ss, _, uu), _ = so.read_forward(
            a["x"], a["h"], a["slots"], a["ages"], a["usage"],
            {k: a[k] for k in P}, cfg)
        return (hh * cot_h).sum() + (ss * cot_s).sum() + (uu * cot_u).sum()

    eps = 1e-6
    for n in names:
        flat = np.array(arrays[n], np.float64).reshape(-1)
        g = grads[n].numpy().reshape(-1)
        for i in range(flat.size):
            a = {k: np.array(v, np.float64) for k, v in arrays.items()}
            f = a[n].reshape(-1)
            f[i] = flat[i] + eps
            a[n] = f.reshape(np.shape(arrays[n]))
            fp = objective(a)
            f[i] = flat[i] - eps
            fm = objective(a)
            fd = (fp - fm) / (2 * eps)
            assert abs(fd - g[i]) < 1e-6 * max(1.0, abs(fd)), (n, i, fd,
                                                                g[i])


def test_pins_catch_planted_mistakes(monkeypatch):
    x, h, slots, ages, usage, P, cfg = _case(seed=5, T=4)
    P0 = dict(P, tau_r_raw=np.array(0.0))
    zero = np.zeros_like(slots)

    # the read taken after the slot update: zero slots no longer read zero
    real = so.read_forward

    def read_after_update(x, h, s, a, u, P, cfg):
        C = x.shape[-1]
        x_ln = so.layer_norm(x, P["ln_scale"], P["ln_bias"])
        dker = P["delta_kernel"]
        delta0 = np.tanh((x_ln[:, 0] @ dker[:C] + h[:, 0] @ dker[C:2 * C])
                         [:, None, :] + P["slot_embed"] @ dker[2 * C:]
                         + P["delta_bias"])
        mu = so.compute_mu(cfg, P["mu_by_bank_raw"])[None, :, None]
        return real(x, h, s + mu * (delta0 - s), a, u, P, cfg)

    bad, _, _ = read_after_update(x, h, zero, ages, usage, P0, cfg)
    assert np.max(np.abs(bad[:, 0] - h[:, 0])) > 1e-6

    # a wrong per-slot rate (its complement) in the numpy oracle: the torch
    # restatement, which derives mu on its own, rejects it
    def bad_compute_mu(cfg, raw):
        return 1.0 - real_mu(cfg, raw)

    real_mu = so.compute_mu
    monkeypatch.setattr(so, "compute_mu", bad_compute_mu)
    h_bad, (s_bad, _, _), _ = so.read_forward(x, h, slots, ages, usage, P,
                                              cfg)
    monkeypatch.undo()
    h_t, s_t, _ = so.read_forward_torch(
        _t(x), _t(h), _t(slots), _t(ages), _t(usage),
        {k: _t(v) for k, v in P.items()}, cfg)
    assert np.max(np.abs(s_bad - s_t.numpy())) > 1e-3
    assert np.max(np.abs(h_bad - h_t.numpy())) > 1e-6


WRITE = dict(use_write_screening=True, write_rel_floor=0.05)


@pytest.mark.parametrize("opt", [dict(), dict(use_age_mask=True)], ids=str)
def test_write_phase_restatements_agree(opt):
    x, h, slots, ages, usage, P, cfg = _case(seed=11, T=7, **WRITE, **opt)
    hn, (sn, an, un), stats = so.read_forward(x, h, slots, ages, usage, P,
                                              cfg, phase="read_write")
    ht, st, ut = so.read_forward_torch(
        _t(x), _t(h), _t(slots), _t(ages), _t(usage),
        {k: _t(v) for k, v in P.items()}, cfg, phase="read_write")
    np.testing.assert_allclose(hn, ht.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(sn, st.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(un, ut.numpy(), rtol=1e-12, atol=1e-13)
    # the write phase changes the slots, ages and statistics
    _, (s_ro, a_ro, _), st_ro = so.read_forward(x, h, slots, ages, usage, P,
                                                cfg)
    assert np.max(np.abs(sn - s_ro)) > 1e-6
    assert np.array_equal(a_ro, ages) and not np.array_equal(an, ages)
    assert stats["rel_write_effective_mean"] >= 0.05 - 1e-12
    assert st_ro["rel_write_mean"] == 0.0 and stats["tau_w"] != 0.0


def test_write_phase_ages_and_floor():
    # ages count steps without a write and reset where rel_w > 1e-3; with a
    # query orthogonal to every write key nothing is written and the
    # strength is the floor: slots move by mu * floor per step
    x, h, slots, ages, usage, P, cfg = _case(seed=12, T=3, **WRITE)
    P0 = dict(P, q_proj_w=np.zeros_like(P["q_proj_w"]),
              tau_w_raw=np.array(0.0))
    _, (s_t, a_t, _), st = so.read_forward(x, h, slots, ages, usage, P0,
                                           cfg, phase="read_write")
    np.testing.assert_allclose(a_t, ages + 3.0)
    assert st["rel_write_mean"] == 0.0
    cfg_ro = dict(cfg, mu_short_max=cfg["mu_short_max"] * 0.05,
                  mu_mid_max=cfg["mu_mid_max"] * 0.05,
                  mu_long_max=cfg["mu_long_max"] * 0.05)
    _, (s_ro, _, _), _ = so.read_forward(x, h, slots, ages, usage, P0,
                                         cfg_ro)
    np.testing.assert_allclose(s_t, s_ro, rtol=1e-12, atol=1e-14)


def test_write_phase_autograd_matches_finite_differences():
    x, h, slots, ages, usage, P, cfg = _case(B=1, T=3, C=4, ds=3, dk=3,
                                             dv=3, M=2, seed=13,
                                             use_age_mask=True, **WRITE)
    rng = np.random.default_rng(130)
    cot_h = rng.normal(size=x.shape)
    cot_s = rng.normal(size=slots.shape)
    cot_u = rng.normal(size=usage.shape)
    names = ["x", "h", "slots", "usage"] + sorted(P)
    arrays = dict(x=x, h=h, slots=slots, usage=usage, **P)
    tin = {k: _t(v, True) for k, v in arrays.items()}
    ht, st, ut = so.read_forward_torch(
        tin["x"], tin["h"], tin["slots"], _t(ages), tin["usage"],
        {k: tin[k] for k in P}, cfg, phase="read_write")
    loss = ((ht * _t(cot_h)).sum() + (st * _t(cot_s)).sum()
            + (ut * _t(cot_u)).sum())
    grads = dict(zip(names, torch.autograd.grad(loss, [tin[n]
                                                       for n in names])))

    def objective(a):
        hh, (ss, _, uu), _ = so.read_forward(
            a["x"], a["h"], a["slots"], ages, a["usage"],
            {k: a[k] for k in P}, cfg, phase="read_write")
        return (hh * cot_h).sum() + (ss * cot_s).sum() + (uu * cot_u).sum()

    eps = 1e-6
    for n in names:
        flat = np.array(arrays[n], np.float64).reshape(-1)
        g = grads[n].numpy().reshape(-1)
        for i in range(flat.size):
            a = {k: np.array(v, np.float64) for k, v in arrays.items()}
            f = a[n].reshape(-1)
            f[i] = flat[i] + eps
            a[n] = f.reshape(np.shape(arrays[n]))
            fp = objective(a)
            f[i] = flat[i] - eps
            fm = objective(a)
            fd = (fp - fm) / (2 * eps)
            assert abs(fd - g[i]) < 1e-6 * max(1.0, abs(fd)), (n, i, fd,
                                                                g[i])


# ---------------------------------------------------------------------------
# Hand-built cases: every quantity below is worked out from the definitions
# (reference screening.py:21-58, nnx_model.py:1062-1137) with numbers chosen
# so that it has a short closed form, not by re-running the oracle's steps.
#
#   x = [3, -1]: LayerNorm mean 1, variance 4, so x_ln = [s, -s] with
#   s = 2 / sqrt(4 + 1e-6); q_proj_r keeps x_ln's first channel, so the read
#   query is e1.  k_proj_r = I and unit slots make the keys the slots; the
#   three slots e1, [0.6, 0.8], e2 then have similarities 1, 0.6, 0.
#   tau_r_raw = log 1.5 gives tau = 2 * 0.6 - 1 = 0.2; lambda_raw =
#   log(e^0.5 - 1) gives lambda = 0.5; v_proj = 2 I, so the unit-normed
#   values are the slots (and twice the slots without the unit norm).
# ---------------------------------------------------------------------------

S_LN = 2.0 / np.sqrt(4.0 + 1e-6)
SLOTS3 = np.array([[1.0, 0.0], [0.6, 0.8], [0.0, 1.0]])
OUT3 = np.array([[1.0, -2.0], [0.5, 3.0]])
DELTA3 = np.tanh(np.array([0.3, -0.2]))
MU3 = np.array([0.05, 0.02, 0.005]) / 2.0     # mu_max * sigmoid(0), banks 0-2
AGES3 = np.array([32.0, 32.0 + 8.0 * np.log(3.0), 0.0])
USAGE3 = np.array([0.1, 0.0, 0.2])


def _hand(T=1, delta_bias=(0.3, -0.2), **opt):
    cfg = so.default_config(d_model=2, d_slot=2, d_k=2, d_v=2, n_slots=3,
                            bank_ids=(0, 1, 2), eps=1e-12, **opt)
    P = {"ln_scale": np.ones(2), "ln_bias": np.zeros(2),
         "q_proj_r": np.array([[1.0, 0.0], [0.0, 0.0]]),
         "k_proj_r": np.eye(2), "v_proj": 2.0 * np.eye(2), "out_proj": OUT3,
         "gate_kernel": np.array([[0.7, 0.0], [0.0, 0.0]]),
         "gate_bias": np.array([0.1, -0.4]),
         "delta_kernel": np.zeros((6, 2)),
         "delta_bias": np.array(delta_bias, np.float64),
         "tau_r_raw": np.array(np.log(1.5)),
         "lambda_raw": np.array(np.log(np.expm1(0.5))),
         "slot_embed": np.zeros((3, 2)), "mu_by_bank_raw": np.zeros(3),
         # write path: the write query is unit(h) = e2 (x's part is zero),
         # the write keys are the slots, tau_w = 0.2 as tau
         "q_proj_w": np.vstack([np.zeros((2, 2)), np.eye(2)]),
         "k_proj_w": np.eye(2), "tau_w_raw": np.array(np.log(1.5))}
    x = np.tile(np.array([3.0, -1.0]), (1, T, 1))
    h = np.tile(np.array([0.0, 2.0]), (1, T, 1))
    return (x, h, SLOTS3[None].copy(), AGES3[None].copy(),
            USAGE3[None].copy(), P, cfg)


def _hand_read(rel, value_scale=1.0):
    """h at a step whose relevances are ``rel``: z = sum_m rel_m v_m,
    u = tanh(|z|) z / |z| (cap 1), h = h_base + lambda * gate * u @ out."""
    z = value_scale * rel @ SLOTS3
    nz = np.linalg.norm(z)
    u = np.tanh(nz) / nz * z
    gate = 1.0 / (1.0 + np.exp(-np.array([0.7 * S_LN + 0.1, -0.4])))
    return np.array([0.0, 2.0]) + 0.5 * gate * (u @ OUT3), z, u


def _check_hand(opt, rel, value_scale=1.0, torch_too=True):
    x, h, slots, ages, usage, P, cfg = _hand(**opt)
    want_h, z, u = _hand_read(rel, value_scale)
    hn, (sn, an, un), stats = so.read_forward(x, h, slots, ages, usage, P,
                                              cfg)
    np.testing.assert_allclose(hn[0, 0], want_h, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(sn[0], SLOTS3 + MU3[:, None]
                               * (DELTA3 - SLOTS3), rtol=1e-9, atol=1e-15)
    np.testing.assert_allclose(un[0], 0.99 * USAGE3 + 0.01 * rel,
                               rtol=1e-9, atol=1e-15)
    np.testing.assert_array_equal(an, ages)
    if torch_too:
        ht, st, ut = so.read_forward_torch(
            _t(x), _t(h), _t(slots), _t(ages), _t(usage),
            {k: _t(v) for k, v in P.items()}, cfg)
        np.testing.assert_allclose(ht.numpy()[0, 0], want_h, rtol=1e-9,
                                   atol=1e-12)
        np.testing.assert_allclose(ut.numpy()[0], un[0], rtol=1e-9)
    return stats, z, u


def test_hand_built_read():
    # trim-square relevances ((sim - 0.2) / 0.8)^2 of 1, 0.6, 0
    _check_hand({}, np.array([1.0, 0.25, 0.0]))
    # a one-hot slot gives z = rel * v: only e1 clears tau = 0.7
    # (tau_r_raw = log(0.85 / 0.15))
    x, h, slots, ages, usage, P, cfg = _hand()
    P["tau_r_raw"] = np.array(np.log(0.85 / 0.15))
    hn, _, stats = so.read_forward(x, h, slots, ages, usage, P, cfg)
    rel = np.array([1.0, 0.0, 0.0])
    want_h, z, _ = _hand_read(rel)
    np.testing.assert_allclose(z, [1.0, 0.0])
    np.testing.assert_allclose(hn[0, 0], want_h, rtol=1e-9)
    assert stats["active_slots_mean"] == 1.0
    # without the value unit norm the values are 2 * slots
    _check_hand(dict(use_value_unit_norm=False), np.array([1.0, 0.25, 0.0]),
                value_scale=2.0)
    # age weights sigmoid((32 - age) / 8): 1/2 at age 32, 1/4 at
    # 32 + 8 ln 3, and e2's relevance is 0 whatever its weight
    _check_hand(dict(use_age_mask=True), np.array([0.5, 0.0625, 0.0]))
    # leaky warm-up: 0.7 * trim (reference eps 1e-6) + 0.3 * sigmoid(8 (sim
    # - tau)); e2 (sim 0, below tau) still reads through the soft term
    hard = np.array([0.8, 0.4, 0.0]) ** 2 / (0.8 + 1e-6) ** 2
    soft = 1.0 / (1.0 + np.exp(-8.0 * np.array([0.8, 0.4, -0.2])))
    _check_hand(dict(use_leaky_warmup=True, leaky_alpha=0.3),
                0.7 * hard + 0.3 * soft)


def test_hand_built_statistics():
    rel = np.array([1.0, 0.25, 0.0])
    stats, z, u = _check_hand({}, rel)
    upd = MU3 * np.linalg.norm(DELTA3 - SLOTS3, axis=-1)
    want = {"rel_read_mean": 1.25 / 3.0, "rel_read_max": 1.0,
            "active_slots_mean": 2.0, "z_norm_mean": np.sqrt(1.3625),
            "u_norm_mean": np.tanh(np.sqrt(1.3625)), "tau_r": 0.2,
            "lambda_screen": 0.5, "rel_write_mean": 0.0,
            "rel_write_effective_mean": 0.0,
            "slot_update_norm_mean": upd.mean(),
            "slot_usage_ema_mean": (0.99 * USAGE3 + 0.01 * rel).mean(),
            "tau_w": 0.0}
    np.testing.assert_allclose(z, [1.15, 0.2])
    assert set(stats) == set(want)
    for k, v in want.items():
        np.testing.assert_allclose(stats[k], v, rtol=1e-9, atol=1e-15,
                                   err_msg=k)


def test_hand_built_steps_average_the_statistics():
    # delta = tanh(0) = 0 shrinks each slot by (1 - mu) per step without
    # turning it, so every step reads the same; the usage follows the EMA in
    # closed form and the update norms are mu (1 - mu)^t
    T = 3
    x, h, slots, ages, usage, P, cfg = _hand(T=T, delta_bias=(0.0, 0.0))
    hn, (sn, _, un), stats = so.read_forward(x, h, slots, ages, usage, P,
                                             cfg)
    rel = np.array([1.0, 0.25, 0.0])
    want_h, _, _ = _hand_read(rel)
    np.testing.assert_allclose(hn[0], np.tile(want_h, (T, 1)), rtol=1e-9)
    np.testing.assert_allclose(sn[0], (1 - MU3[:, None]) ** T * SLOTS3,
                               rtol=1e-9)
    usage_t = [0.99 ** t * USAGE3 + (1 - 0.99 ** t) * rel
               for t in range(1, T + 1)]
    np.testing.assert_allclose(un[0], usage_t[-1], rtol=1e-9)
    np.testing.assert_allclose(stats["slot_usage_ema_mean"],
                               np.mean([u.mean() for u in usage_t]),
                               rtol=1e-9)
    np.testing.assert_allclose(
        stats["slot_update_norm_mean"],
        np.mean([(MU3 * (1 - MU3) ** t).mean() for t in range(T)]),
        rtol=1e-9)
    np.testing.assert_allclose(stats["rel_read_mean"], 1.25 / 3.0,
                               rtol=1e-9)


def test_hand_built_write():
    # write query e2 against the slots: similarities 0, 0.8, 1, so with
    # tau_w = 0.2 the write relevances are 0, 0.5625, 1; e1 is written at
    # the floor and ages, the others reset to age 0
    x, h, slots, ages, usage, P, cfg = _hand(use_write_screening=True,
                                             write_rel_floor=0.05)
    hn, (sn, an, un), stats = so.read_forward(x, h, slots, ages, usage, P,
                                              cfg, phase="read_write")
    rel = np.array([1.0, 0.25, 0.0])
    rel_w = np.array([0.0, 0.5625, 1.0])
    strength = MU3 * np.maximum(rel_w, 0.05)
    want_h, _, _ = _hand_read(rel)
    np.testing.assert_allclose(hn[0, 0], want_h, rtol=1e-9)
    np.testing.assert_allclose(
        sn[0], SLOTS3 + strength[:, None] * (DELTA3 - SLOTS3), rtol=1e-9,
        atol=1e-14)
    np.testing.assert_array_equal(an[0], [AGES3[0] + 1.0, 0.0, 0.0])
    activity = np.array([1.0, 0.5625, 1.0])
    np.testing.assert_allclose(un[0], 0.99 * USAGE3 + 0.01 * activity,
                               rtol=1e-9)
    np.testing.assert_allclose(stats["rel_write_mean"], 1.5625 / 3.0,
                               rtol=1e-9)
    np.testing.assert_allclose(stats["rel_write_effective_mean"],
                               1.6125 / 3.0, rtol=1e-9)
    np.testing.assert_allclose(stats["tau_w"], 0.2, rtol=1e-9)
    np.testing.assert_allclose(
        stats["slot_update_norm_mean"],
        (strength * np.linalg.norm(DELTA3 - SLOTS3, axis=-1)).mean(),
        rtol=1e-9)
    ht, st, ut = so.read_forward_torch(
        _t(x), _t(h), _t(slots), _t(ages), _t(usage),
        {k: _t(v) for k, v in P.items()}, cfg, phase="read_write")
    np.testing.assert_allclose(ht.numpy(), hn, rtol=1e-9)
    np.testing.assert_allclose(st.numpy(), sn, rtol=1e-9)
    np.testing.assert_allclose(ut.numpy(), un, rtol=1e-9)


def test_half_life_rates():
    # a half-life H gives the rate mu with (1 - mu)^H = 1/2; banks without
    # one keep mu_max * sigmoid(raw)
    cfg = so.default_config(short_half_life_tokens=4.0,
                            long_half_life_tokens=50.0, bank_ids=(0, 1, 2))
    mu = so.compute_mu(cfg, np.array([5.0, np.log(3.0), -5.0]))
    np.testing.assert_allclose((1.0 - mu[[0, 2]]) ** np.array([4.0, 50.0]),
                               0.5, rtol=1e-13)
    np.testing.assert_allclose(mu[1], 0.02 * 0.75, rtol=1e-13)


@pytest.mark.parametrize("plant", ["no_squash", "no_square", "exp_lambda",
                                   "gate_without_sigmoid", "no_layer_norm"])
def test_hand_pins_catch_planted_mistakes(monkeypatch, plant):
    if plant == "no_squash":
        monkeypatch.setattr(so, "tanh_norm", lambda z, cap, eps: z)
    elif plant == "no_square":
        monkeypatch.setattr(so, "trim_square", lambda s, t, e: np.maximum(
            (s - t) / (1.0 - t + e), 0.0))
    elif plant == "exp_lambda":
        monkeypatch.setattr(so, "softplus", np.exp)
    elif plant == "gate_without_sigmoid":   # the only [B, T, C] sigmoid
        real = so.sigmoid
        monkeypatch.setattr(so, "sigmoid",
                            lambda v: v if np.ndim(v) == 3 else real(v))
    else:   # gate and query fed the raw input: the gate sees 3, not ~1
        monkeypatch.setattr(so, "layer_norm", lambda x, sc, b, eps=1e-6: x)
    with pytest.raises(AssertionError):
        _check_hand({}, np.array([1.0, 0.25, 0.0]), torch_too=False)


def _scalar_grads(case, cfg_opt_cots, n):
    """float64 autograd gradient of the loss sum(cot * output) with respect
    to the scalar parameter n, and the sum of its terms' magnitudes."""
    x, h, slots, ages, usage, P, cfg = case
    cot_h, cot_s, cot_u = cfg_opt_cots
    arrays = dict(x=x, h=h, slots=slots, ages=ages, usage=usage, **P)
    base = {k: _t(v) for k, v in arrays.items()}

    def f(theta):
        a = dict(base)
        a[n] = theta
        return so.read_forward_torch(a["x"], a["h"], a["slots"], a["ages"],
                                     a["usage"], {k: a[k] for k in P}, cfg)

    theta = base[n].clone().requires_grad_(True)
    ht, st, ut = f(theta)
    loss = ((ht * _t(cot_h)).sum() + (st * _t(cot_s)).sum()
            + (ut * _t(cot_u)).sum())
    (g,) = torch.autograd.grad(loss, [theta])
    _, jac = torch.autograd.functional.jvp(f, base[n],
                                           torch.ones_like(base[n]))
    scale = float(sum((j * _t(c)).abs().sum()
                      for j, c in zip(jac, (cot_h, cot_s, cot_u))))
    return float(g), scale


@pytest.mark.parametrize("opt", [dict(), dict(use_age_mask=True)], ids=str)
def test_scalar_gradient_measures_reject_planted_errors(opt):
    # The GPU parity tests measure a scalar parameter's gradient with
    # so.scalar_grad_error: fp32 against its own magnitude (1e-4), bf16
    # against the sum of its terms' magnitudes (4e-3), because such a
    # gradient is a sum over every output element that cancels heavily
    # (|grad| / sum|terms| = 0.006 .. 0.07 at the GPU tests' shapes).
    # Planted errors in tau_r_raw's oracle gradient (it cancels most) show
    # what each measure rejects.  fp32 rejects every one: a dropped group of
    # terms (the usage EMA's path, one token's h outputs) and a relative
    # error above 1e-4.  Under the bf16 measure a relative error d reads as
    # d * ratio and a dropped group as its share of sum|terms|, rejected
    # above 4e-3: the usage path is, a single token's outputs (0.3 % of the
    # terms in the first case) may not be.  The screening kernels run the
    # same code for both compute dtypes, so such algorithmic mistakes are
    # the fp32 checks' to catch; the bf16 checks bound the bf16 roundings.
    case = _case(B=2, T=23, C=64, ds=80, dk=32, dv=80, M=5,
                 seed=7 + len(str(opt)), **opt)
    x, h, slots, ages, usage, P, cfg = case
    rng = np.random.default_rng(3)
    cots = (rng.normal(size=x.shape), rng.normal(size=slots.shape),
            rng.normal(size=usage.shape))
    want, scale = _scalar_grads(case, cots, "tau_r_raw")
    ratio = abs(want) / scale
    print(f"  {opt}: dtau_r_raw {want:.4e}, sum|terms| {scale:.4e}, "
          f"ratio {ratio:.3e}")
    assert 1e-4 < ratio < 0.2  # heavy cancellation, as on the GPU
    t32, t16 = so.SCALAR_TOL_FP32, so.SCALAR_TOL_BF16

    def measures(got):
        e32, _, b32, s32 = so.scalar_grad_error(got, want, scale, True)
        e16, r, b16, s16 = so.scalar_grad_error(got, want, scale, False)
        assert (b32, b16) == ("own magnitude", "terms")
        assert (s32, s16) == (t32, t16)
        assert r == pytest.approx(ratio)
        return e32, e16

    # dropped groups of terms: the usage EMA's path, the last token's h
    dropped_usage, _ = _scalar_grads(case, (cots[0], cots[1], 0 * cots[2]),
                                     "tau_r_raw")
    cot_h = cots[0].copy()
    cot_h[:, -1] = 0.0
    dropped_token, _ = _scalar_grads(case, (cot_h,) + cots[1:], "tau_r_raw")
    for what, got in (("usage path", dropped_usage),
                      ("last token", dropped_token)):
        e32, e16 = measures(got)
        print(f"  {opt}: {what} dropped: fp32 error {e32:.3e}, bf16 error "
              f"{e16:.3e} (the group's share of sum|terms|)")
        assert e32 > t32, what
        assert e16 == pytest.approx(abs(got - want) / scale)
    assert measures(dropped_usage)[1] > t16
    # relative errors: the terms measure reads d * ratio
    for d in (0.5 * t16 / ratio, 1.5 * t16 / ratio):
        _, e16 = measures(want * (1 + d))
        assert e16 == pytest.approx(d * ratio, rel=1e-9)
        assert (e16 > t16) == (d > t16 / ratio)
    for d, rejected in ((0.5 * t32, False), (1.5 * t32, True), (0.05, True)):
        e32, _ = measures(want * (1 + d))
        assert (e32 > t32) == rejected, d
    # a gradient that cancelled by more than 1000x is measured against its
    # terms in fp32 too, where d * ratio must stay below 1e-6
    tiny = 0.5 * so.HEAVY_CANCELLATION * scale
    e, r, basis, tol = so.scalar_grad_error(tiny * (1 + 0.01), tiny, scale,
                                            True)
    assert (basis, tol) == ("terms", so.SCALAR_TOL_FP32_TERMS)
    assert e == pytest.approx(0.01 * r) and e > tol
