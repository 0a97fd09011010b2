"""Pins for the CPU oracle (CPU only).

Every oracle function is checked against something other than its own
formula: the reference's numpy known-answer test, closed forms, an explicit
transition-matrix formulation, torch float64 autograd, central finite
differences, and the reference's checkpoint-format test. A planted-mistake
test shows that the pins catch a transposed operand and a dropped term.
"""

import numpy as np
import pytest
import torch

import oracle

RNG_SHAPES = [(1, 1, 1, 4), (5, 1, 2, 4), (9, 2, 3, 8), (17, 1, 2, 16)]


def _rand_inputs(shape, seed, scale=1.0, s0_scale=0.3):
    rng = np.random.default_rng(seed)
    T, B, H, N = shape
    r, w, k, v, a, b = (rng.normal(size=shape) * scale for _ in range(6))
    s0 = rng.normal(size=(B, H, N, N)) * s0_scale
    return r, w, k, v, a, b, s0


# ---------------------------------------------------------------------------
# Reference known-answer test: tests/test_upstream_rwkv7_parity.py:265-297
# ---------------------------------------------------------------------------

def test_reference_known_answer_single_step():
    rng = np.random.default_rng(19)
    n = 4
    state = rng.normal(size=(1, 1, n, n)).astype(np.float32)
    r = rng.normal(size=(1, 1, n)).astype(np.float32)
    raw_w = rng.normal(size=(1, 1, n)).astype(np.float32)
    k = rng.normal(size=(1, 1, n)).astype(np.float32)
    v = rng.normal(size=(1, 1, n)).astype(np.float32)
    a = rng.normal(size=(1, 1, n)).astype(np.float32)
    b = rng.normal(size=(1, 1, n)).astype(np.float32)
    # The reference test's own expected values (official CUDA row update).
    decay = np.exp(-np.exp(raw_w))
    sa = np.einsum("bhij,bhj->bhi", state, a)
    expected_state = (state * decay[..., None, :]
                      + np.einsum("bhi,bhj->bhij", sa, b)
                      + np.einsum("bhi,bhj->bhij", v, k))
    expected_y = np.einsum("bhij,bhj->bhi", expected_state, r)

    vecs = [x[None] for x in (r, raw_w, k, v, a, b)]
    for impl in ("c64", "c32", "np"):
        if impl == "np":
            y, s = oracle.np_forward(*vecs, state)
        else:
            y, s = oracle.forward(*vecs, state,
                                  precision="f64" if impl == "c64" else "f32")
        np.testing.assert_allclose(s, expected_state, atol=1e-6, rtol=1e-6)
        np.testing.assert_allclose(y[0], expected_y, atol=1e-6, rtol=1e-6)


# ---------------------------------------------------------------------------
# Closed forms and invariants of the forward
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", RNG_SHAPES)
def test_pure_decay_closed_form(shape):
    r, w, k, v, a, b, s0 = _rand_inputs(shape, 1)
    zeros = np.zeros(shape)
    y, s_t = oracle.forward(r, w, zeros, zeros, zeros, b, s0)
    # S_t = S0 * prod_{u<=t} d_u[j]  ->  log-space cumulative sum
    logp = -np.cumsum(np.exp(w), axis=0)                       # [T,B,H,N]
    states = s0[None] * np.exp(logp)[..., None, :]
    np.testing.assert_allclose(s_t, states[-1], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(
        y, np.einsum("tbhij,tbhj->tbhi", states, r), rtol=1e-10, atol=1e-13)


@pytest.mark.parametrize("shape", RNG_SHAPES)
def test_no_decay_running_outer_product_sum(shape):
    r, w, k, v, a, b, s0 = _rand_inputs(shape, 2)
    w = np.full(shape, -60.0)          # exp(-exp(-60)) == 1.0 in float64
    zeros = np.zeros(shape)
    y, s_t = oracle.forward(r, w, k, v, zeros, zeros, s0)
    outer = np.einsum("tbhi,tbhj->tbhij", v, k)
    states = s0[None] + np.cumsum(outer, axis=0)
    np.testing.assert_allclose(s_t, states[-1], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(
        y, np.einsum("tbhij,tbhj->tbhi", states, r), rtol=1e-10, atol=1e-12)


def _transition_forward(r, w, k, v, a, b, s0):
    """S_t = S_{t-1} @ (diag(d_t) + a_t b_t^T) + v_t k_t^T with explicit
    N x N transition matrices (a different formulation of rwkv_core.py:54-86
    that fixes which side a and b act on)."""
    s = np.array(s0, np.float64)
    ys = []
    for t in range(r.shape[0]):
        d = np.exp(-np.exp(w[t]))
        m = np.einsum("bhj,jl->bhjl", d, np.eye(d.shape[-1])) + \
            a[t][..., :, None] * b[t][..., None, :]
        s = s @ m + v[t][..., :, None] * k[t][..., None, :]
        ys.append(s @ r[t][..., :, None])
    return np.stack(ys)[..., 0], s


@pytest.mark.parametrize("shape", RNG_SHAPES)
def test_forward_matches_transition_matrix_formulation(shape):
    inputs = _rand_inputs(shape, 3, scale=0.7)
    y_ref, s_ref = _transition_forward(*inputs)
    for y, s in (oracle.forward(*inputs), oracle.np_forward(*inputs)):
        np.testing.assert_allclose(y, y_ref, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(s, s_ref, rtol=1e-10, atol=1e-12)


def test_single_step_equals_t1_and_rows_are_independent():
    shape = (6, 2, 2, 8)
    r, w, k, v, a, b, s0 = _rand_inputs(shape, 4)
    y, s_t = oracle.forward(r, w, k, v, a, b, s0)
    # T=1 pieces chained by hand equal the scan
    s = s0
    for t in range(shape[0]):
        y1, s = oracle.forward(*(x[t:t + 1] for x in (r, w, k, v, a, b)), s)
        np.testing.assert_allclose(y1[0], y[t], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s, s_t, rtol=1e-12, atol=1e-12)
    # permuting state rows and v permutes y and S_T rows the same way
    perm = np.random.default_rng(5).permutation(shape[-1])
    yp, sp = oracle.forward(r, w, k, v[..., perm], a, b, s0[..., perm, :])
    np.testing.assert_allclose(yp, y[..., perm], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sp, s_t[..., perm, :], rtol=1e-12, atol=1e-12)


def test_c_and_numpy_restatements_agree():
    inputs = _rand_inputs((13, 2, 3, 8), 6, scale=0.8)
    y1, s1 = oracle.forward(*inputs)
    y2, s2 = oracle.np_forward(*inputs)
    assert np.max(np.abs(y1 - y2)) < 1e-11
    assert np.max(np.abs(s1 - s2)) < 1e-11
    y3, s3 = oracle.forward(*inputs, precision="f32", threads=2)
    assert oracle.normalized_max_error(y3, y1) < 1e-5
    assert oracle.normalized_max_error(s3, s1) < 1e-5


def test_checkpoint_format_matches_reference_aux_contract():
    # tests/test_wkv_pallas.py:84-108: T=5, interval 2 -> (4,1,2,4,4) and the
    # last checkpoint equals the final state even for a partial interval.
    inputs = _rand_inputs((5, 1, 2, 4), 17, scale=0.1, s0_scale=0.1)
    y, s_t, ckpt = oracle.forward(*inputs, checkpoint_interval=2)
    assert ckpt.shape == (4, 1, 2, 4, 4)
    _, _, states, _ = oracle.np_forward(*inputs, return_states=True)
    np.testing.assert_allclose(ckpt[0], inputs[-1])
    np.testing.assert_allclose(ckpt[1], states[2], rtol=1e-12)
    np.testing.assert_allclose(ckpt[2], states[4], rtol=1e-12)
    np.testing.assert_allclose(ckpt[-1], s_t, rtol=1e-12)


# ---------------------------------------------------------------------------
# Backward: torch float64 autograd and finite differences
# ---------------------------------------------------------------------------

def _torch_transition_forward(r, w, k, v, a, b, s0):
    s = s0
    ys = []
    n = r.shape[-1]
    eye = torch.eye(n, dtype=torch.float64)
    for t in range(r.shape[0]):
        d = torch.exp(-torch.exp(w[t]))
        m = d[..., :, None] * eye + a[t][..., :, None] * b[t][..., None, :]
        s = s @ m + v[t][..., :, None] * k[t][..., None, :]
        ys.append((s @ r[t][..., :, None])[..., 0])
    return torch.stack(ys), s


@pytest.mark.parametrize("shape", [(1, 1, 1, 4), (5, 1, 2, 4), (20, 2, 2, 8),
                                   (33, 1, 1, 16)])
def test_backward_matches_torch_autograd(shape):
    inputs = _rand_inputs(shape, 7, scale=0.6)
    rng = np.random.default_rng(8)
    dy = rng.normal(size=shape)
    ds_t = rng.normal(size=inputs[-1].shape) * 0.5
    tin = [torch.tensor(x, dtype=torch.float64, requires_grad=True)
           for x in inputs]
    y, s = _torch_transition_forward(*tin)
    loss = (y * torch.tensor(dy)).sum() + (s * torch.tensor(ds_t)).sum()
    expected = torch.autograd.grad(loss, tin)
    for got in (oracle.backward(*inputs, dy, ds_t),
                oracle.np_backward(*inputs, dy, ds_t)):
        for g, e in zip(got, expected):
            np.testing.assert_allclose(g, e.numpy(), rtol=1e-9, atol=1e-11)
    got32 = oracle.backward(*inputs, dy, ds_t, precision="f32", threads=2)
    for g, e in zip(got32, expected):
        assert oracle.normalized_max_error(g, e.numpy()) < 2e-5


def test_backward_matches_central_finite_differences():
    shape = (4, 1, 1, 4)
    inputs = [np.array(x) for x in _rand_inputs(shape, 9, scale=0.5)]
    rng = np.random.default_rng(10)
    dy = rng.normal(size=shape)
    ds_t = rng.normal(size=inputs[-1].shape)

    def objective(vals):
        y, s = oracle.forward(*vals)
        return float(np.sum(y * dy) + np.sum(s * ds_t))

    grads = oracle.backward(*inputs, dy, ds_t)
    eps = 1e-6
    for idx, (x, g) in enumerate(zip(inputs, grads)):
        flat = x.reshape(-1)
        for p in range(flat.size):
            orig = flat[p]
            flat[p] = orig + eps
            fp = objective(inputs)
            flat[p] = orig - eps
            fm = objective(inputs)
            flat[p] = orig
            fd = (fp - fm) / (2 * eps)
            assert abs(fd - g.reshape(-1)[p]) < 1e-6 * max(1.0, abs(fd)), (
                idx, p, fd, g.reshape(-1)[p])


# ---------------------------------------------------------------------------
# bf16 helper and the pins' own sensitivity
# ---------------------------------------------------------------------------

def test_bf16_rounding_is_round_to_nearest_even():
    vals = np.array([1.0, -2.5, 3.1415927, 1e-30, 65504.0, np.inf, -np.inf],
                    np.float32)
    bits = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x00000001],
                    np.uint32).view(np.float32)
    x = np.concatenate([vals, bits,
                        np.random.default_rng(11).normal(size=1000)
                        .astype(np.float32)])
    expected = torch.tensor(x).to(torch.bfloat16).view(torch.int16).numpy()
    np.testing.assert_array_equal(oracle.bf16_bits(x),
                                  expected.view(np.uint16))
    assert oracle.bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0
    assert oracle.bf16_bits(np.array([0x3F808000], np.uint32)
                            .view(np.float32))[0] == 0x3F80
    assert oracle.bf16_bits(np.array([0x3F818000], np.uint32)
                            .view(np.float32))[0] == 0x3F82


def test_pins_catch_planted_mistakes():
    """Plant a transposed operand and a dropped term in a copy of the numpy
    oracle and check the transition-matrix and autograd pins reject it."""
    inputs = _rand_inputs((6, 1, 2, 8), 12, scale=0.7)
    y_ref, s_ref = _transition_forward(*inputs)
    r, w, k, v, a, b, s0 = inputs
    # transposed low-rank update: b and a swapped
    y_bad, s_bad = oracle.np_forward(r, w, k, v, b, a, s0)
    assert np.max(np.abs(s_bad - s_ref)) > 1e-3
    # dropped v k^T term
    y_bad, s_bad = oracle.np_forward(r, w, np.zeros_like(k), v, a, b, s0)
    assert np.max(np.abs(y_bad - y_ref)) > 1e-3
    # backward with a sign error in the decay derivative
    rng = np.random.default_rng(13)
    dy = rng.normal(size=r.shape)
    ds_t = np.zeros_like(s0)
    good = oracle.np_backward(*inputs, dy, ds_t)
    tin = [torch.tensor(x, dtype=torch.float64, requires_grad=True)
           for x in inputs]
    yt, st = _torch_transition_forward(*tin)
    exp_dw = torch.autograd.grad((yt * torch.tensor(dy)).sum(), tin[1])[0]
    np.testing.assert_allclose(good[1], exp_dw.numpy(), rtol=1e-9, atol=1e-11)
    assert np.max(np.abs(-good[1] - exp_dw.numpy())) > 1e-3
