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
* planted mistakes fail those pins: the read taken after the slot update
  (zero slots then read something), and a wrong per-slot rate in the numpy
  restatement (the torch restatement, which derives the rates on its own,
  disagrees).
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
