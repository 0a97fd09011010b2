"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle
and the committed golden fixtures.

Tolerances (the path's accuracy targets): fp32 inputs -- max|diff| / max|oracle|
<= 1e-4 per tensor; bf16 inputs with an fp32 state -- <= 2e-2 of the
oracle's max magnitude per tensor. The oracle is float64 on the same inputs.
"""

import glob
import os

import numpy as np
import pytest
import torch

import oracle
from rwkv7m_amd.synthetic import config_inputs, make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")
GRAD_NAMES = ("dr", "dw", "dk", "dv", "dneg_kk", "dkka", "ds0")
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _to_dev(inputs):
    return {k: v.cuda() for k, v in inputs.items()}


def _assert_close(name, got, expected, tol, case=""):
    err = oracle.normalized_max_error(_np(got) if torch.is_tensor(got)
                                      else got, expected)
    assert err <= tol, f"{case} {name}: normalized max error {err:.3e} > {tol}"


def _oracle_all(inp):
    vecs = [_np(inp[n]) for n in NAMES]
    s0 = _np(inp["s0"])
    y, s_t = oracle.forward(*vecs, s0)
    grads = oracle.backward(*vecs, s0, _np(inp["dy"]), _np(inp["ds_t"]))
    return y, s_t, grads


def _run_hip(hip, inp, ci=0):
    vecs = [inp[n] for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, inp["s0"],
                                         checkpoint_interval=ci)
    grads = hip.backward(*vecs, inp["s0"], inp["dy"], inp["ds_t"], *aux)
    y2, s_t2 = hip.forward(*vecs, inp["s0"])
    torch.cuda.synchronize()
    return y, s_t, aux, grads, y2, s_t2


def test_config0_fp32_forward_matches_oracle(hip):
    inp = _to_dev(config_inputs(0))
    print("case: config 0 fp32 forward B2 T64 H4 N16", flush=True)
    vecs = [inp[n] for n in NAMES]
    y, s_t = hip.forward(*vecs, inp["s0"])
    torch.cuda.synchronize()
    ey, es = oracle.forward(*[_np(inp[n]) for n in NAMES], _np(inp["s0"]))
    assert y.dtype == torch.float32 and s_t.dtype == torch.float32
    _assert_close("y", y, ey, 1e-4)
    _assert_close("s_t", s_t, es, 1e-4)


CASES = [
    # (T, B, H, N, state_std, dstate_std)
    (3, 1, 2, 4, 0.1, 0.1),
    (5, 1, 2, 4, 0.1, 0.0),
    (37, 2, 3, 16, 0.1, 0.1),
    (70, 2, 2, 64, 0.0, 0.0),
    (41, 1, 2, 64, 0.1, 0.1),
    (20, 1, 1, 128, 0.03, 0.03),
    (9, 1, 3, 1, 0.1, 0.1),
    (9, 1, 1, 2, 0.1, 0.1),
    (33, 2, 1, 8, 0.1, 0.1),
    (16, 1, 2, 32, 0.1, 0.1),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_forward_backward_match_oracle(hip, case, dtype):
    T, B, H, N, sstd, dsstd = case
    tag = f"T{T} B{B} H{H} N{N} {dtype}"
    print("case:", tag, flush=True)
    inp = make_inputs(T, B, H, N, dtype=dtype, seed=T * 131 + N,
                      state_std=sstd, dstate_std=dsstd)
    ey, es, egrads = _oracle_all(inp)
    y, s_t, aux, grads, y2, s_t2 = _run_hip(hip, _to_dev(inp))
    tol = TOL[dtype]
    assert y.dtype == dtype and s_t.dtype == torch.float32
    _assert_close("y", y, ey, tol, tag)
    _assert_close("s_t", s_t, es, tol, tag)
    _assert_close("y(forward)", y2, ey, tol, tag)
    _assert_close("s_t(forward)", s_t2, es, tol, tag)
    for name, g, e in zip(GRAD_NAMES, grads, egrads):
        assert g.dtype == (torch.float32 if name == "ds0" else dtype)
        _assert_close(name, g, e, tol, tag)


@pytest.mark.parametrize("n", [32, 64, 128])
def test_sequential_backward_saved_states_long_interval(hip, n):
    """One interval of 300 tokens: the sequential backward's sub-interval
    start states are saved in LDS several at a time (16 at N = 32, 6 at
    N = 64, 3 at N = 128 over two row-split workgroups); every grouping (the
    partial group first), the partial last sub-interval and the prefetched
    vector blocks against the oracle."""
    print("case: sequential backward, T = 300, interval 256, N =", n,
          flush=True)
    inp = make_inputs(300, 1, 2, n, dtype=torch.float32, seed=91,
                      state_std=0.1, dstate_std=0.1)
    ey, es, egrads = _oracle_all(inp)
    y, s_t, aux, grads, _, _ = _run_hip(hip, _to_dev(inp), ci=256)
    assert aux[0].shape[0] == 3
    _assert_close("y", y, ey, 1e-4, f"N={n}")
    _assert_close("s_t", s_t, es, 1e-4, f"N={n}")
    for name, g, e in zip(GRAD_NAMES, grads, egrads):
        _assert_close(name, g, e, 1e-4, f"N={n}")


def test_sequential_backward_row_split_time_segments(hip):
    """N = 128 splits each head's rows over two workgroups, whose shares of
    the column sums (dr, dw, dk, da, db) a second kernel adds; the shares of
    8 heads fit 3264 tokens at a time, so 3500 tokens run as two time
    segments that pass dS through dS0."""
    print("case: sequential backward, B2 T3500 H4 N128, interval 16",
          flush=True)
    inp = make_inputs(3500, 2, 4, 128, dtype=torch.float32, seed=93,
                      state_std=0.1, dstate_std=0.1)
    ey, es, egrads = _oracle_all(inp)
    y, s_t, aux, grads, _, _ = _run_hip(hip, _to_dev(inp), ci=16)
    _assert_close("y", y, ey, 1e-4, "N=128")
    _assert_close("s_t", s_t, es, 1e-4, "N=128")
    for name, g, e in zip(GRAD_NAMES, grads, egrads):
        _assert_close(name, g, e, 1e-4, "N=128")


@pytest.mark.parametrize("ci", [1, 3, 16, 64, 200])
def test_checkpoint_interval_does_not_change_results(hip, ci):
    print("case: checkpoint interval", ci, flush=True)
    inp = make_inputs(70, 1, 2, 64, dtype=torch.float32, seed=77,
                      state_std=0.1, dstate_std=0.1)
    ey, es, egrads = _oracle_all(inp)
    y, s_t, aux, grads, _, _ = _run_hip(hip, _to_dev(inp), ci=ci)
    assert aux[0].shape[0] == (70 + ci - 1) // ci + 1
    _assert_close("y", y, ey, 1e-4)
    for name, g, e in zip(GRAD_NAMES, grads, egrads):
        _assert_close(name, g, e, 1e-4, f"ci={ci}")


def test_aux_checkpoint_format(hip):
    # reference tests/test_wkv_pallas.py:84-108
    print("case: aux format T5 ci2", flush=True)
    inp = _to_dev(make_inputs(5, 1, 2, 4, dtype=torch.float32, seed=17,
                              state_std=0.1))
    vecs = [inp[n] for n in NAMES]
    (y, s_t), (ckpt, ci) = hip.forward_with_aux(*vecs, inp["s0"],
                                                checkpoint_interval=2)
    torch.cuda.synchronize()
    assert int(ci) == 2
    assert tuple(ckpt.shape) == (4, 1, 2, 4, 4)
    _, _, eck = oracle.forward(*[_np(inp[n]) for n in NAMES],
                               _np(inp["s0"]), checkpoint_interval=2)
    assert torch.equal(ckpt[0], inp["s0"])
    assert torch.equal(ckpt[-1], s_t)
    _assert_close("checkpoints", ckpt, eck, 1e-5)


def test_decode_inplace_matches_oracle_over_steps(hip):
    print("case: decode 16 steps B4 H3 N64 bf16", flush=True)
    B, H, N, steps = 4, 3, 64, 16
    inp = make_inputs(steps, B, H, N, seed=5, state_std=0.1)
    ey, es = oracle.forward(*[_np(inp[n]) for n in NAMES], _np(inp["s0"]))
    dev = _to_dev(inp)
    state = dev["s0"].clone()
    ptr = state.data_ptr()
    ys = []
    for t in range(steps):
        ys.append(hip.decode_inplace(*(dev[n][t] for n in NAMES), state))
    torch.cuda.synchronize()
    assert state.data_ptr() == ptr
    _assert_close("y", torch.stack(ys), ey, 2e-2)
    _assert_close("state", state, es, 2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16],
                         ids=["f32", "bf16"])
def test_decode_kernel_many_heads(hip, dtype):
    """The single-token kernel (N = 64) at 1024 heads, in place, against
    the oracle; then against the sequential kernel on the same step (a
    T = 1 forward with checkpoints takes the sequential kernel)."""
    print(f"case: decode B64 H16 N64 {dtype}", flush=True)
    inp = make_inputs(1, 64, 16, 64, dtype=dtype, seed=21, state_std=0.1)
    ey, es = oracle.forward(*[_np(inp[n]) for n in NAMES], _np(inp["s0"]))
    dev = _to_dev(inp)
    state = dev["s0"].clone()
    y = hip.decode_inplace(*(dev[n][0] for n in NAMES), state)
    torch.cuda.synchronize()
    _assert_close("y", y[None], ey, TOL[dtype])
    _assert_close("state", state, es, 1e-5)
    (ys, ss), _ = hip.forward_with_aux(*(dev[n] for n in NAMES), dev["s0"],
                                       checkpoint_interval=1)
    torch.cuda.synchronize()
    _assert_close("y vs sequential", y[None], _np(ys), TOL[dtype])
    _assert_close("state vs sequential", state, _np(ss), 1e-6)


def test_decode_kernel_closed_form(hip):
    """d = 1 (w -> -inf) and a = b = 0: one step is S + v k^T exactly
    enough to compare at fp32 rounding, and y = (S + v k^T) r."""
    print("case: decode closed form B3 H5 N64 f32", flush=True)
    g = torch.Generator().manual_seed(22)
    B, H, N = 3, 5, 64
    s0 = torch.randn(B, H, N, N, generator=g)
    k = torch.randn(1, B, H, N, generator=g)
    v = torch.randn(1, B, H, N, generator=g)
    r = torch.randn(1, B, H, N, generator=g)
    w = torch.full((1, B, H, N), -1e4)
    z = torch.zeros(1, B, H, N)
    es = (s0.double() + v[0].double()[..., :, None] * k[0].double()[..., None, :])
    ey = torch.einsum("bhij,bhj->bhi", es, r[0].double())
    state = s0.cuda()
    y = hip.decode_inplace(*(x.cuda() for x in (r, w, k, v, z, z)), state)
    torch.cuda.synchronize()
    _assert_close("state", state, es.numpy(), 1e-6)
    _assert_close("y", y[0], ey.numpy(), 1e-5)


def test_forward_state_in_place_alias(hip):
    print("case: forward with out_state aliasing S0", flush=True)
    inp = _to_dev(make_inputs(9, 2, 2, 64, seed=6, state_std=0.1))
    vecs = [inp[n] for n in NAMES]
    y_ref, s_ref = hip.forward(*vecs, inp["s0"])
    state = inp["s0"].clone()
    y, s = hip.forward(*vecs, state, out_state=state)
    torch.cuda.synchronize()
    assert s.data_ptr() == state.data_ptr()
    assert torch.equal(y, y_ref) and torch.equal(state, s_ref)


def test_empty_time_axis(hip):
    print("case: T=0", flush=True)
    inp = _to_dev(make_inputs(0, 2, 2, 16, seed=7, state_std=0.1,
                              dstate_std=0.1))
    vecs = [inp[n] for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, inp["s0"])
    grads = hip.backward(*vecs, inp["s0"], inp["dy"], inp["ds_t"], *aux)
    torch.cuda.synchronize()
    assert y.shape == (0, 2, 2, 16)
    assert torch.equal(s_t, inp["s0"])
    assert torch.equal(grads[-1], inp["ds_t"])
    assert all(g.numel() == 0 for g in grads[:-1])


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN,
                                                               "*.npz"))),
                         ids=os.path.basename)
def test_golden_fixtures(hip, path):
    print("case: golden", os.path.basename(path), flush=True)
    data = np.load(path)
    bf16 = bool(data["is_bf16"])
    dtype = torch.bfloat16 if bf16 else torch.float32

    def vec(name):
        x = data[name]
        if bf16:
            x = oracle.bf16_from_bits(x)
        return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()

    inp = {n: vec(n) for n in NAMES}
    inp["s0"] = torch.from_numpy(data["s0"]).cuda()
    tol = TOL[dtype]
    vecs = [inp[n] for n in NAMES]
    if "dr" in data:
        inp["dy"] = vec("dy")
        inp["ds_t"] = torch.from_numpy(data["ds_t"]).cuda()
        y, s_t, aux, grads, _, _ = _run_hip(hip, inp)
        for name, g in zip(GRAD_NAMES, grads):
            _assert_close(name, g, data[name], tol, path)
    else:
        y, s_t = hip.forward(*vecs, inp["s0"])
        torch.cuda.synchronize()
    _assert_close("y", y, data["y"], tol, path)
    _assert_close("s_t", s_t, data["s_t"], tol, path)


def test_c_abi_rejects_bad_requests_without_launching(hip):
    lib = hip.load_library()
    null = [None] * 10
    assert lib.rwkv7m_wkv7_forward(5, 1, 1, 1, 4, *null) == 1
    assert b"bfloat16 or float32" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_forward(0, 1, 1, 1, 48, *null) == 2
    assert lib.rwkv7m_wkv7_forward(0, 2, 1, 1, 4, *null) == 1
    assert b"is NULL" in lib.rwkv7m_last_error()
    x = torch.zeros(3, 1, 1, 4, device="cuda")
    with pytest.raises(RuntimeError, match="GPU tensors"):
        hip.forward(*(x.cpu() for _ in range(6)),
                    torch.zeros(1, 1, 4, 4))
