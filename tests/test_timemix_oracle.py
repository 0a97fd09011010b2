"""Pins for the time-mix producer/consumer oracle (CPU only).

``oracle/timemix_oracle.py`` restates nnx_model.py:630, :683-694 and
:709-727.  Each of its functions is checked against something other than
its own formula:

* the forwards against torch.nn.functional library routines in float64
  (``softplus``, ``normalize``, ``group_norm``) on the same inputs;
* invariants: every head of kk has unit norm; GroupNorm with unit scale and
  zero bias gives zero mean and variance var / (var + eps) per head;
* the clamp's asymptotes (w -> -0.5 for large w_raw, w -> w_raw - 0.5 for
  very negative w_raw) and its range (w < -0.5);
* the backwards against float64 torch autograd of the library forms and
  against central finite differences of the oracle forwards, for every
  activation and parameter cotangent;
* planted mistakes (a dropped mean^2 in the variance, k' taken after the
  normalisation, a dropped term of da) fail those same checks.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import timemix_oracle as tmo

SHAPES = [(1, 1, 8), (5, 2, 8), (7, 3, 16), (4, 2, 64)]  # rows, H, N


def _inputs(rows, H, N, seed):
    rng = np.random.default_rng(seed)
    C = H * N
    act = {n: rng.normal(size=(rows, C)) for n in
           ("w_raw", "k", "y", "r", "v", "g")}
    act["w_raw"] = act["w_raw"] * 2.0 - 1.0
    act["a"] = 1.0 / (1.0 + np.exp(-rng.normal(size=(rows, C))))
    par = {"k_k": 0.7 + 0.1 * rng.normal(size=C),
           "k_a": 1.0 + 0.05 * rng.normal(size=C),
           "r_k": -0.04 + 0.3 * rng.normal(size=C),
           "scale": 0.5 + rng.random(size=C),
           "bias": 0.2 * rng.normal(size=C)}
    return act, par


def _t(x, grad=False):
    return torch.tensor(x, dtype=torch.float64, requires_grad=grad)


# ---------------------------------------------------------------------------
# torch library forms (float64)
# ---------------------------------------------------------------------------

def _lib_inputs(w_raw, k, a, k_k, k_a, N):
    rows, C = k.shape
    w = -F.softplus(-w_raw, beta=1.0, threshold=1e4) - 0.5
    kk = F.normalize((k * k_k).reshape(rows, C // N, N), dim=-1,
                     eps=1e-300).reshape(rows, C)
    kp = k * (1.0 + (a - 1.0) * k_a)
    return w, kp, -kk, kk * a


def _lib_output(y, r, k, v, g, r_k, scale, bias, N, eps):
    rows, C = y.shape
    gn = F.group_norm(y, C // N, scale, bias, eps)
    s = (r * k * r_k).reshape(rows, C // N, N).sum(-1, keepdim=True)
    bonus = (s * v.reshape(rows, C // N, N)).reshape(rows, C)
    return (gn + bonus) * g


@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_inputs_forward_matches_library_routines(rows, H, N):
    act, par = _inputs(rows, H, N, 1)
    got = tmo.wkv_inputs(act["w_raw"], act["k"], act["a"], par["k_k"],
                         par["k_a"], N)
    want = _lib_inputs(*(_t(x) for x in (act["w_raw"], act["k"], act["a"],
                                         par["k_k"], par["k_a"])), N)
    for g_, w_ in zip(got, want):
        np.testing.assert_allclose(g_, w_.numpy(), rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_output_forward_matches_library_routines(rows, H, N):
    act, par = _inputs(rows, H, N, 2)
    args = [act[n] for n in ("y", "r", "k", "v", "g")] + \
        [par[n] for n in ("r_k", "scale", "bias")]
    got = tmo.wkv_output(*args, N, eps=64e-5)
    want = _lib_output(*(_t(x) for x in args), N, 64e-5)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_invariants_and_asymptotes():
    act, par = _inputs(9, 3, 16, 3)
    w, kp, nkk, kka = tmo.wkv_inputs(act["w_raw"], act["k"], act["a"],
                                     par["k_k"], par["k_a"], 16)
    norms = np.sqrt((nkk.reshape(9, 3, 16) ** 2).sum(-1))
    np.testing.assert_allclose(norms, 1.0, rtol=1e-13)
    np.testing.assert_allclose(kka, -nkk * act["a"], rtol=1e-15)
    assert np.all(w < -0.5)
    x = np.array([[40.0, -40.0, 0.0, 3.0, -3.0, 100.0, -100.0, 1e-3]])
    ones = np.ones((1, 8))
    w, _, _, _ = tmo.wkv_inputs(x, ones, ones, ones[0], ones[0], 8)
    np.testing.assert_allclose(w[0, :2], [-0.5, -40.5], atol=1e-15)
    np.testing.assert_allclose(w[0, 2], -np.log(2.0) - 0.5, rtol=1e-15)
    np.testing.assert_allclose(w[0, 5:7], [-0.5, -100.5], atol=1e-15)
    # a zero head stays zero (the 1e-24 floor keeps the division finite)
    _, _, nkk0, _ = tmo.wkv_inputs(x, np.zeros((1, 8)), ones, ones[0],
                                   ones[0], 8)
    assert np.all(nkk0 == 0.0)
    # GroupNorm with unit scale, zero bias: zero mean, var/(var+eps)
    y = act["y"] * 3.0 + 1.5
    zeros = np.zeros_like(y)
    out = tmo.wkv_output(y, zeros, zeros, zeros, np.ones_like(y),
                         np.zeros(48), np.ones(48), np.zeros(48), 16,
                         eps=64e-5)
    yh = y.reshape(9, 3, 16)
    var = yh.var(-1)
    oh = out.reshape(9, 3, 16)
    np.testing.assert_allclose(oh.mean(-1), 0.0, atol=1e-13)
    np.testing.assert_allclose(oh.var(-1), var / (var + 64e-5), rtol=1e-12)


# ---------------------------------------------------------------------------
# Backward: torch autograd of the library forms and finite differences
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_inputs_backward_matches_torch_autograd(rows, H, N):
    act, par = _inputs(rows, H, N, 4)
    rng = np.random.default_rng(40)
    cots = [rng.normal(size=act["k"].shape) for _ in range(4)]
    names = ("w_raw", "k", "a")
    tin = [_t(act[n], True) for n in names] + \
        [_t(par[n], True) for n in ("k_k", "k_a")]
    outs = _lib_inputs(*tin, N)
    loss = sum((o * _t(c)).sum() for o, c in zip(outs, cots))
    want = torch.autograd.grad(loss, tin)
    got = tmo.wkv_inputs_backward(act["w_raw"], act["k"], act["a"],
                                  par["k_k"], par["k_a"], *cots, N)
    for g_, w_ in zip(got, want):
        np.testing.assert_allclose(g_, w_.numpy(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_output_backward_matches_torch_autograd(rows, H, N):
    act, par = _inputs(rows, H, N, 5)
    dout = np.random.default_rng(50).normal(size=act["y"].shape)
    tin = [_t(act[n], True) for n in ("y", "r", "k", "v", "g")] + \
        [_t(par[n], True) for n in ("r_k", "scale", "bias")]
    out = _lib_output(*tin, N, 64e-5)
    want = torch.autograd.grad((out * _t(dout)).sum(), tin)
    got = tmo.wkv_output_backward(*(x.detach().numpy() for x in tin), dout,
                                  N, eps=64e-5)
    for g_, w_ in zip(got, want):
        np.testing.assert_allclose(g_, w_.numpy(), rtol=1e-9, atol=1e-11)


def _fd_check(fn, bwd, arrays, cot, tol=1e-6):
    """Central differences of sum(fn(arrays) * cot) against bwd."""
    grads = bwd
    h = 1e-6
    for idx, (x, g) in enumerate(zip(arrays, grads)):
        flat = x.reshape(-1)
        for p in range(flat.size):
            orig = flat[p]
            flat[p] = orig + h
            fp = sum(np.sum(o * c) for o, c in zip(fn(arrays), cot))
            flat[p] = orig - h
            fm = sum(np.sum(o * c) for o, c in zip(fn(arrays), cot))
            flat[p] = orig
            fd = (fp - fm) / (2 * h)
            assert abs(fd - g.reshape(-1)[p]) < tol * max(1.0, abs(fd)), (
                idx, p, fd, g.reshape(-1)[p])


def test_inputs_backward_matches_finite_differences():
    act, par = _inputs(3, 2, 8, 6)
    arrays = [act["w_raw"].copy(), act["k"].copy(), act["a"].copy(),
              par["k_k"].copy(), par["k_a"].copy()]
    rng = np.random.default_rng(60)
    cots = [rng.normal(size=act["k"].shape) for _ in range(4)]
    bwd = tmo.wkv_inputs_backward(*arrays, *cots, 8)
    _fd_check(lambda a: tmo.wkv_inputs(*a, 8), bwd, arrays, cots)


def test_output_backward_matches_finite_differences():
    act, par = _inputs(3, 2, 8, 7)
    arrays = [act[n].copy() for n in ("y", "r", "k", "v", "g")] + \
        [par[n].copy() for n in ("r_k", "scale", "bias")]
    dout = np.random.default_rng(70).normal(size=act["y"].shape)
    bwd = tmo.wkv_output_backward(*arrays, dout, 8, eps=64e-5)
    _fd_check(lambda a: (tmo.wkv_output(*a, 8, eps=64e-5),), bwd, arrays,
              (dout,))


# ---------------------------------------------------------------------------
# The pins' own sensitivity: mistakes planted in copies of the oracle
# ---------------------------------------------------------------------------

def test_pins_catch_planted_mistakes(monkeypatch):
    act, par = _inputs(5, 2, 16, 8)
    args = [act[n] for n in ("y", "r", "k", "v", "g")] + \
        [par[n] for n in ("r_k", "scale", "bias")]
    want = _lib_output(*(_t(x) for x in args), 16, 64e-5).numpy()

    # variance without the mean^2 term
    def bad_gn(y, scale, bias, N, eps):
        yh = y.reshape(y.shape[0], -1, N)
        mean = yh.mean(-1, keepdims=True)
        rstd = 1.0 / np.sqrt((yh * yh).mean(-1, keepdims=True) + eps)
        xhat = ((yh - mean) * rstd).reshape(y.shape)
        return xhat * scale + bias, xhat, rstd

    with monkeypatch.context() as m:
        m.setattr(tmo, "_group_norm", bad_gn)
        bad = tmo.wkv_output(*[a + 1.0 if i == 0 else a
                               for i, a in enumerate(args)], 16)
    want_shift = _lib_output(*(_t(a + 1.0 if i == 0 else a)
                               for i, a in enumerate(args)), 16,
                             64e-5).numpy()
    assert np.max(np.abs(bad - want_shift)) > 1e-3
    np.testing.assert_allclose(tmo.wkv_output(*args, 16), want, rtol=1e-10,
                               atol=1e-12)

    # k' computed from the normalised kk instead of k
    lib = _lib_inputs(*(_t(x) for x in (act["w_raw"], act["k"], act["a"],
                                        par["k_k"], par["k_a"])), 16)
    _, _, nkk, _ = tmo.wkv_inputs(act["w_raw"], act["k"], act["a"],
                                  par["k_k"], par["k_a"], 16)
    bad_kp = -nkk * (1.0 + (act["a"] - 1.0) * par["k_a"])
    assert np.max(np.abs(bad_kp - lib[1].numpy())) > 1e-3

    # da missing its dkka * kk term
    rng = np.random.default_rng(80)
    cots = [rng.normal(size=act["k"].shape) for _ in range(4)]
    good = tmo.wkv_inputs_backward(act["w_raw"], act["k"], act["a"],
                                   par["k_k"], par["k_a"], *cots, 16)
    bad_da = good[2] - cots[3] * -nkk
    tin = [_t(act[n], True) for n in ("w_raw", "k", "a")] + \
        [_t(par[n]) for n in ("k_k", "k_a")]
    outs = _lib_inputs(*tin, 16)
    loss = sum((o * _t(c)).sum() for o, c in zip(outs, cots))
    exp_da = torch.autograd.grad(loss, tin[2])[0].numpy()
    np.testing.assert_allclose(good[2], exp_da, rtol=1e-10, atol=1e-12)
    assert np.max(np.abs(bad_da - exp_da)) > 1e-3
