"""GPU parity of the chunked MFMA kernels (bf16 vectors, N = 64) against the
float64 CPU oracle.

The MFMA path serves bf16 inputs with head size 64 and the checkpoint
intervals in MFMA_INTERVALS; any other interval runs the sequential kernels.
Every case asserts which kernels served it (rwkv7m_wkv7_last_path), so a
case is labelled by the path it provably took.  Tolerance (the bf16 bound
of the path's accuracy target): max|diff| <= 2e-2 * max|oracle| per tensor.  Cases cover partial
final chunks, every interval, nonzero initial state and state cotangent, and
decays strong enough to force the in-kernel exact sequential fallback.
"""

import numpy as np
import pytest
import torch

import oracle
from rwkv7m_amd.synthetic import config_inputs, make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")
GRAD_NAMES = ("dr", "dw", "dk", "dv", "dneg_kk", "dkka", "ds0")
TOL = 2e-2
THREADS = 8
# checkpoint intervals the MFMA kernels serve (both directions)
MFMA_INTERVALS = (16, 32, 64)


def expected_paths(ci):
    """(forward, backward) kernel paths of a bf16 N = 64 training call."""
    if ci in MFMA_INTERVALS:
        return ("wave_forward", "wave_backward")
    return ("seq_forward", "seq_backward")


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _check(name, got, expected, case, tol=TOL):
    err = oracle.normalized_max_error(_np(got), expected)
    assert err <= tol, f"{case} {name}: normalized max error {err:.3e} > {tol}"
    return err


def _run_case(hip, inp, ci, case, check_grads=True):
    """ci is passed to the library as is (0: its default); the checks use
    the interval in effect."""
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                         checkpoint_interval=ci)
    paths = [hip.last_path()]
    grads = None
    if check_grads:
        grads = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux)
        paths.append(hip.last_path())
    torch.cuda.synchronize()
    hip.device_status()
    eff = ci or hip.default_checkpoint_interval(torch.bfloat16, 64)
    assert tuple(paths) == expected_paths(eff)[:len(paths)], (case, paths)
    host = [_np(inp[n]) for n in NAMES]
    ey, es, eck = oracle.forward(*host, _np(inp["s0"]),
                                 checkpoint_interval=eff, threads=THREADS)
    assert y.dtype == torch.bfloat16 and s_t.dtype == torch.float32
    _check("y", y, ey, case)
    _check("s_t", s_t, es, case)
    # checkpoints in the library's dtype for this interval (bf16 on every
    # MFMA interval): S0 and S_T rounded to nearest even
    cdt = hip.checkpoint_dtype(torch.bfloat16, 64, ci)
    assert aux[0].dtype == cdt
    if eff in MFMA_INTERVALS:
        assert cdt == torch.bfloat16
    _check("checkpoints", aux[0], eck, case)
    assert torch.equal(aux[0][0], dev["s0"].to(cdt))
    assert torch.equal(aux[0][-1], s_t.to(cdt))
    if check_grads:
        egr = oracle.backward(*host, _np(inp["s0"]), _np(inp["dy"]),
                              _np(inp["ds_t"]), threads=THREADS)
        for name, g, e in zip(GRAD_NAMES, grads, egr):
            _check(name, g, e, case)


@pytest.mark.parametrize("ci", [16, 32, 64])
@pytest.mark.parametrize("T", [2, 17, 64, 100, 130])
def test_chunked_matches_oracle(hip, T, ci):
    case = f"chunked T{T} B2 H2 N64 L{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(T, 2, 2, 64, seed=900 + T + ci, state_std=0.1,
                      dstate_std=0.1)
    _run_case(hip, inp, ci, case)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_chunked_strong_decay_uses_exact_fallback(hip, ci):
    # exp(w) ~ 7 per token: every chunk exceeds the factored form's range
    case = f"strong decay T80 L{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(80, 1, 3, 64, seed=31 + ci, state_std=0.1,
                      dstate_std=0.1)
    g = torch.Generator().manual_seed(5)
    inp["w"] = (torch.randn(inp["w"].shape, generator=g) + 2.0).to(
        torch.bfloat16)
    _run_case(hip, inp, ci, case)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_chunked_mixed_fast_and_fallback_chunks(hip, ci):
    # decay strong only in tokens 64..127 of head 1: chunks there take the
    # exact fallback, the rest the MFMA path, and the state crosses both
    case = f"mixed decay T192 L{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(192, 2, 2, 64, seed=44, state_std=0.1, dstate_std=0.1)
    w = inp["w"].float()
    w[64:128, :, 1] += 3.0
    inp["w"] = w.to(torch.bfloat16)
    _run_case(hip, inp, ci, case)


def test_chunked_unit_decay_and_tiny_inputs(hip):
    # w -> -inf (decay exactly 1): the running outer-product sum
    case = "unit decay T70 L32"
    print("case:", case, flush=True)
    inp = make_inputs(70, 1, 2, 64, seed=8, state_std=0.1, dstate_std=0.1)
    inp["w"] = torch.full_like(inp["w"], -30.0)
    inp["neg_kk"] = torch.zeros_like(inp["neg_kk"])
    inp["kka"] = torch.zeros_like(inp["kka"])
    _run_case(hip, inp, 32, case)


def test_chunked_plain_forward_and_in_place_state(hip):
    case = "plain forward T150 (library default chunk)"
    print("case:", case, flush=True)
    inp = make_inputs(150, 2, 3, 64, seed=12, state_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    y, s_t = hip.forward(*vecs, dev["s0"])
    state = dev["s0"].clone()
    y2, _ = hip.forward(*vecs, state, out_state=state)
    torch.cuda.synchronize()
    ey, es = oracle.forward(*[_np(inp[n]) for n in NAMES], _np(inp["s0"]))
    _check("y", y, ey, case)
    _check("s_t", s_t, es, case)
    assert torch.equal(y, y2) and torch.equal(state, s_t)


def test_config1_forward_backward_default_path(hip):
    # config 1 in full on the library's default (MFMA) path, interval 0
    # (the library default, 16), and at interval 32
    assert hip.default_checkpoint_interval(torch.bfloat16, 64) == 16
    inp = config_inputs(1)
    for ci in (0, 32):
        case = f"config 1: B8 T512 H12 N64 bf16 L{ci or 'default'}"
        print("case:", case, flush=True)
        _run_case(hip, inp, ci, case)


def test_config1_forward_backward_sequential_kernels(hip):
    # an interval outside MFMA_INTERVALS runs the sequential kernels
    case = "config 1: B8 T512 H12 N64 bf16 L128 (sequential kernels)"
    print("case:", case, flush=True)
    inp = config_inputs(1)
    _run_case(hip, inp, 128, case)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_config4_distributions_slow_decay_carry_state(hip, ci):
    # config 4's distributions (slow decay, S0 and dS_T ~ N(0, 0.1)) on a
    # reduced (B, H) at T = 2048; the full size is in
    # test_fullsize_parity.py
    case = f"config 4 distributions B1 T2048 H2 N64 L{ci}"
    print("case:", case, flush=True)
    inp = config_inputs(4, T=2048, B=1, H=2)
    _run_case(hip, inp, ci, case)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_chunked_results_are_deterministic(hip, ci):
    # The same inputs must give bit-identical outputs on every call: each
    # workgroup owns one (batch, head) and reduces in a fixed order.
    case = f"determinism T320 B4 H8 L{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(320, 4, 8, 64, seed=77 + ci, state_std=0.1,
                      dstate_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    first = None
    for _ in range(6):
        (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                             checkpoint_interval=ci)
        fwd_path = hip.last_path()
        grads = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux)
        assert (fwd_path, hip.last_path()) == expected_paths(ci)
        outs = [y, s_t, aux[0], *grads]
        torch.cuda.synchronize()
        if first is None:
            first = [o.clone() for o in outs]
        else:
            for name, a_, b_ in zip(("y", "s_t", "ckpt") + GRAD_NAMES, first,
                                    outs):
                assert torch.equal(a_, b_), f"{case}: {name} differs"


def _misaligned(t):
    """A copy of t whose data starts 2 bytes past a 16-byte boundary."""
    flat = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    out = flat[1:1 + t.numel()].view(t.shape)
    out.copy_(t)
    return out


def test_sequential_kernels_share_the_bf16_checkpoint_format(hip):
    # Misaligned vectors take the sequential kernels, which then write and
    # read the same bf16 checkpoints as the chunked ones.
    case = "misaligned T70 B1 H2 N64 L32"
    print("case:", case, flush=True)
    inp = make_inputs(70, 1, 2, 64, seed=31, state_std=0.1, dstate_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [_misaligned(dev[n]) for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                         checkpoint_interval=32)
    grads = hip.backward(*vecs, dev["s0"], _misaligned(dev["dy"]),
                         dev["ds_t"], *aux)
    # the aligned (chunked) forward feeding the misaligned backward, and
    # the misaligned forward feeding the chunked backward
    (y2, _), aux2 = hip.forward_with_aux(*[dev[n] for n in NAMES], dev["s0"],
                                         checkpoint_interval=32)
    grads2 = hip.backward(*[dev[n] for n in NAMES], dev["s0"], dev["dy"],
                          dev["ds_t"], *aux)
    grads3 = hip.backward(*vecs, dev["s0"], _misaligned(dev["dy"]),
                          dev["ds_t"], *aux2)
    torch.cuda.synchronize()
    assert aux[0].dtype == torch.bfloat16
    assert torch.equal(aux[0][0], dev["s0"].to(torch.bfloat16))
    assert torch.equal(aux[0][-1], s_t.to(torch.bfloat16))
    host = [_np(inp[n]) for n in NAMES]
    ey, es, eck = oracle.forward(*host, _np(inp["s0"]),
                                 checkpoint_interval=32, threads=THREADS)
    egr = oracle.backward(*host, _np(inp["s0"]), _np(inp["dy"]),
                          _np(inp["ds_t"]), threads=THREADS)
    _check("y", y, ey, case)
    _check("s_t", s_t, es, case)
    _check("checkpoints", aux[0], eck, case)
    _check("checkpoints(chunked)", aux2[0], eck, case)
    for gs, tag in ((grads, ""), (grads2, " chunked bwd"),
                    (grads3, " seq bwd of chunked fwd")):
        for name, g, e in zip(GRAD_NAMES, gs, egr):
            _check(name, g, e, case + tag)


def test_empty_time_axis_bf16_checkpoints(hip):
    print("case: T=0 B2 H2 N64 bf16", flush=True)
    inp = make_inputs(0, 2, 2, 64, seed=8, state_std=0.1, dstate_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"])
    grads = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux)
    torch.cuda.synchronize()
    assert aux[0].shape == (1, 2, 2, 64, 64)
    assert torch.equal(aux[0][0], dev["s0"].to(torch.bfloat16))
    assert torch.equal(s_t, dev["s0"])
    assert torch.equal(grads[-1], dev["ds_t"])


def test_operator_api_through_registered_hip_backend(hip):
    # wkv7(..., "ffi") with the HIP kernels registered: the custom VJP's
    # residuals are the library's bf16 checkpoints (reference
    # tests/test_wkv_pallas.py:151-198 with the native backend)
    from rwkv7m_amd.kernels.wkv_ffi import unregister_wkv_ffi_backend
    from rwkv7m_amd.wkv import wkv7
    case = "wkv7 ffi T70 B2 H2 N64"
    print("case:", case, flush=True)
    inp = make_inputs(70, 2, 2, 64, seed=41, state_std=0.1, dstate_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    unregister_wkv_ffi_backend()
    hip.register_hip_backend()
    try:
        xs = [dev[n].clone().requires_grad_(True) for n in (*NAMES, "s0")]
        y, s_t = wkv7(*xs, "ffi")
        grads = torch.autograd.grad((y, s_t), xs,
                                    grad_outputs=(dev["dy"], dev["ds_t"]))
        with torch.no_grad():
            y2, s_t2 = wkv7(*[dev[n] for n in (*NAMES, "s0")], "ffi")
        torch.cuda.synchronize()
    finally:
        unregister_wkv_ffi_backend()
    host = [_np(inp[n]) for n in NAMES]
    ey, es = oracle.forward(*host, _np(inp["s0"]), threads=THREADS)
    egr = oracle.backward(*host, _np(inp["s0"]), _np(inp["dy"]),
                          _np(inp["ds_t"]), threads=THREADS)
    for name, got in (("y", y), ("s_t", s_t), ("y(no grad)", y2),
                      ("s_t(no grad)", s_t2)):
        _check(name, got, ey if name.startswith("y") else es, case)
    for name, g, e in zip(GRAD_NAMES, grads, egr):
        assert g.dtype == (torch.float32 if name == "ds0" else torch.bfloat16)
        _check(name, g, e, case)
