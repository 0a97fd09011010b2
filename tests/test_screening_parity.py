"""GPU parity of the screening read path (``rwkv7m_amd.screening``, HIP
kernels ``rwkv7m_screen_*`` of include/rwkv7m_screening.h) against the
oracle: the float64 numpy scan for the forward and statistics, float64 torch
autograd of the same scan for every gradient (oracle/screening_oracle.py,
restating src/rwkv7m/model/nnx_model.py:999-1160).

Tolerances, normalised max error (max |got - want| / max |want|): 1e-4 for
fp32 activations and parameters, 2e-2 for bf16 activations (compute dtype
bf16, as the reference's presets run), per tensor, forward and backward (the
bf16 oracle runs on the bf16-rounded activations); the gradient of a scalar
parameter (a sum over every output element) is measured against its own
magnitude in fp32 (1e-4; 1e-6 of the terms' sum where the sum cancelled by
more than 1000x, which happens), and against the sum of its terms'
magnitudes in bf16 (4e-3) (oracle.screening_oracle.scalar_grad_error;
tests/test_screening_oracle.py plants errors to show what each measure
rejects).  Shapes include partial
64-channel waves (d_slot = 80, d_v = 80), d_k < 64, several slot counts,
every option of the read (age mask, leaky warm-up, values not normalised,
half-life rates) and the 0.3B preset's sizes.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import screening_oracle as so

pytestmark = pytest.mark.gpu

OPTIONS = [dict(), dict(use_age_mask=True),
           dict(use_leaky_warmup=True, leaky_alpha=0.3),
           dict(use_value_unit_norm=False),
           dict(short_half_life_tokens=4.0, long_half_life_tokens=50.0)]
PNAME = {"ln_scale": "screen_ln_scale", "ln_bias": "screen_ln_bias"}


def _case(B, T, C, ds, dk, dv, M, seed, **opt):
    rng = np.random.default_rng(seed + 1000)
    wparams = {"q_proj_w": rng.normal(size=(2 * C, dk)) / np.sqrt(2 * C),
               "k_proj_w": rng.normal(size=(ds, dk)) / np.sqrt(ds),
               "tau_w_raw": np.array(-1.2)}
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
         "delta_kernel": rng.normal(size=(2 * C + ds, ds)) / np.sqrt(2 * C),
         "delta_bias": 0.1 * rng.normal(size=ds),
         "tau_r_raw": np.array(-1.0), "lambda_raw": np.array(0.3),
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


def _module(P, cfg, dtype):
    from rwkv7m_amd.screening import ScreeningConfig, StateLevelScreening
    mod = StateLevelScreening(ScreeningConfig(**cfg), compute_dtype=dtype,
                              device="cuda")
    with torch.no_grad():
        for k, v in P.items():
            getattr(mod, PNAME.get(k, k)).copy_(torch.tensor(v))
    return mod


def _rnd(a, dtype):
    """Values as the device holds them (bf16 activations are rounded)."""
    return torch.tensor(a, dtype=torch.float32).to(dtype).double().numpy()


def _err(got, want):
    return oracle.normalized_max_error(
        got.detach().double().cpu().numpy(), np.asarray(want, np.float64))


def _run(case, dtype, grad=False, phase="read_screening_only"):
    from rwkv7m_amd.screening import ScreenState
    x, h, slots, ages, usage, P, cfg = case
    mod = _module(P, cfg, dtype)
    xd = torch.tensor(x, dtype=torch.float32).to(dtype).cuda()
    hd = torch.tensor(h, dtype=torch.float32).to(dtype).cuda()
    st = ScreenState(*(torch.tensor(a, dtype=torch.float32).cuda()
                       for a in (slots, ages, usage)))
    if grad:
        xd.requires_grad_(True)
        hd.requires_grad_(True)
        st = ScreenState(*(t.requires_grad_(True) for t in st))
    out, new, stats = mod(xd, hd, st, phase=phase)
    return mod, xd, hd, st, out, new, stats


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("opt", OPTIONS, ids=str)
def test_forward_matches_oracle(hip_lib, opt, dtype):
    case = _case(2, 37, 64, 80, 32, 80, 5, seed=len(str(opt)), **opt)
    name = f"screening fwd {opt} {dtype}"
    print("case:", name, flush=True)
    _, _, _, _, out, new, stats = _run(case, dtype)
    torch.cuda.synchronize()
    x, h, slots, ages, usage, P, cfg = case
    eh, (es, _, eu), est = so.read_forward(_rnd(x, dtype), _rnd(h, dtype),
                                           slots, ages, usage, P, cfg)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for n, g, w in (("h", out, eh), ("slots_T", new.slots, es),
                    ("usage_T", new.usage_ema, eu)):
        e = _err(g, w)
        assert e <= tol, f"{name} {n}: {e:.3e} > {tol}"
    for k in so.STAT_NAMES:
        g, w = float(stats[k]), est[k]
        assert abs(g - w) <= tol * max(1.0, abs(w)), f"{name} stat {k}"
    assert torch.equal(new.ages, torch.tensor(ages, dtype=torch.float32,
                                              device="cuda"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("opt", OPTIONS, ids=str)
def test_backward_matches_autograd_oracle(hip_lib, opt, dtype):
    case = _case(2, 23, 64, 80, 32, 80, 5, seed=7 + len(str(opt)), **opt)
    _check_backward(case, f"screening bwd {opt} {dtype}", dtype)


def _check_backward(case, name, dtype, phase="read_screening_only"):
    print("case:", name, flush=True)
    mod, xd, hd, st, out, new, _ = _run(case, dtype, grad=True, phase=phase)
    x, h, slots, ages, usage, P, cfg = case
    rng = np.random.default_rng(3)
    cot_h = rng.normal(size=x.shape)
    cot_s = rng.normal(size=slots.shape)
    cot_u = rng.normal(size=usage.shape)
    loss = ((out * torch.tensor(cot_h, dtype=torch.float32,
                                device="cuda")).sum()
            + (new.slots * torch.tensor(cot_s, dtype=torch.float32,
                                        device="cuda")).sum()
            + (new.usage_ema * torch.tensor(cot_u, dtype=torch.float32,
                                            device="cuda")).sum())
    loss.backward()
    torch.cuda.synchronize()
    arrays = dict(x=_rnd(x, dtype), h=_rnd(h, dtype), slots=slots, ages=ages,
                  usage=usage, **P)
    tin = {k: torch.tensor(np.asarray(v, np.float64), requires_grad=True)
           for k, v in arrays.items()}
    ht, s_t, u_t = so.read_forward_torch(
        tin["x"], tin["h"], tin["slots"], tin["ages"], tin["usage"],
        {k: tin[k] for k in P}, cfg, phase=phase)
    ref_loss = ((ht * torch.tensor(cot_h)).sum()
                + (s_t * torch.tensor(cot_s)).sum()
                + (u_t * torch.tensor(cot_u)).sum())
    names = list(arrays)
    want = dict(zip(names, torch.autograd.grad(ref_loss,
                                               [tin[n] for n in names],
                                               allow_unused=True)))
    got = {"x": xd.grad, "h": hd.grad, "slots": st.slots.grad,
           "ages": st.ages.grad, "usage": st.usage_ema.grad}
    got.update({k: getattr(mod, PNAME.get(k, k)).grad for k in P})
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for n in names:
        w = want[n]
        if w is None or not np.any(w.numpy()):
            assert got[n] is None or not torch.any(got[n]), f"{name} d{n}"
            continue
        assert got[n] is not None, f"{name} d{n} missing"
        if w.dim() == 0:
            # a scalar parameter's gradient is a sum over every output
            # element that cancels heavily (|grad| / sum|terms| is 2e-5 to
            # 0.12 in these cases): fp32 is measured against its own
            # magnitude unless it cancelled by more than 1000x, bf16 against
            # the sum of its terms' magnitudes (so.scalar_grad_error); the
            # ratio is printed for every case
            scale = _term_scale(tin, n, P, cfg, phase, (cot_h, cot_s, cot_u))
            e, ratio, basis, stol = so.scalar_grad_error(
                float(got[n]), float(w), scale, dtype == torch.float32)
            print(f"  {name} d{n}: |grad| / sum|terms| = {ratio:.3e}, "
                  f"error {e:.3e} against {basis} (tol {stol})", flush=True)
            assert e <= stol, f"{name} d{n}: {e:.3e} > {stol}"
            continue
        else:
            e = _err(got[n], w.numpy())
        assert e <= tol, f"{name} d{n}: {e:.3e} > {tol}"


def _term_scale(tin, n, P, cfg, phase, cots):
    """sum |cot * d(output)/d(theta)| over every output element, for the
    scalar parameter theta = tin[n] (forward-mode derivative of the oracle,
    float64)."""
    base = {k: v.detach() for k, v in tin.items()}

    def f(theta):
        a = dict(base)
        a[n] = theta
        return so.read_forward_torch(a["x"], a["h"], a["slots"], a["ages"],
                                     a["usage"], {k: a[k] for k in P}, cfg,
                                     phase=phase)

    _, jac = torch.autograd.functional.jvp(f, base[n],
                                           torch.ones_like(base[n]))
    return float(sum((j * torch.tensor(c)).abs().sum()
                     for j, c in zip(jac, cots)))


def test_preset_sizes_forward(hip_lib):
    # 0.3B preset: d_model 1024, d_slot 256, d_k 64, d_v 128, 16 slots
    case = _case(2, 48, 1024, 256, 64, 128, 16, seed=11)
    print("case: screening preset 0.3b bf16", flush=True)
    _, _, _, _, out, new, _ = _run(case, torch.bfloat16)
    torch.cuda.synchronize()
    x, h, slots, ages, usage, P, cfg = case
    eh, (es, _, eu), _ = so.read_forward(_rnd(x, torch.bfloat16),
                                         _rnd(h, torch.bfloat16), slots,
                                         ages, usage, P, cfg)
    for n, g, w in (("h", out, eh), ("slots_T", new.slots, es),
                    ("usage_T", new.usage_ema, eu)):
        assert _err(g, w) <= 2e-2, n


def test_phases(hip_lib):
    from rwkv7m_amd.screening import normalize_phase
    case = _case(1, 4, 64, 64, 32, 64, 3, seed=2)
    mod, xd, hd, st, out, _, _ = _run(case, torch.float32)
    out2, _, _ = mod(xd, hd, st, phase="read_only")
    assert torch.equal(out, out2)
    assert normalize_phase("read_only") == "read_screening_only"
    with pytest.raises(ValueError, match="Unknown phase"):
        mod(xd, hd, st, phase="write_only")
    # read_write without write screening is the read-only call
    out3, _, _ = mod(xd, hd, st, phase="read_write")
    assert torch.equal(out, out3)
    # write screening switched on after construction: no write parameters
    mod.config.use_write_screening = True
    with pytest.raises(ValueError, match="write parameters"):
        mod(xd, hd, st, phase="read_write")



@pytest.mark.parametrize("pieces", [(1,) * 6, (33, 1, 37), (70, 1)])
def test_streaming_with_carried_state_equals_one_call(hip_lib, pieces):
    # the reference's generate loop feeds tokens in pieces with the screen
    # state carried (infer/generate.py:62-99): h and the final state of the
    # pieces must equal those of one call over the whole sequence (fp32; the
    # chunked scan composes the steps in another order, so to rounding)
    from rwkv7m_amd.screening import ScreenState
    T = sum(pieces)
    case = _case(2, T, 64, 80, 32, 80, 5, seed=21, use_age_mask=True)
    print("case: screening streaming", pieces, flush=True)
    x, h, slots, ages, usage, P, cfg = case
    mod, xd, hd, st, out, new, _ = _run(case, torch.float32)
    state = st
    outs = []
    t0 = 0
    for n in pieces:
        o, state, _ = mod(xd[:, t0:t0 + n], hd[:, t0:t0 + n], state)
        outs.append(o)
        t0 += n
    torch.cuda.synchronize()
    assert isinstance(state, ScreenState)
    for name, a, b in (("h", torch.cat(outs, 1), out),
                       ("slots", state.slots, new.slots),
                       ("usage", state.usage_ema, new.usage_ema)):
        e = _err(a, b.detach().double().cpu().numpy())
        assert e <= 1e-5, f"streaming {pieces} {name}: {e:.3e}"


@pytest.mark.parametrize("phase", ["read_screening_only", "read_write"])
def test_graph_capture_replays_match_eager(hip_lib, phase):
    # forward + backward captured in one HIP graph (the launch-bound step's
    # deployment form) and replayed three times, with unrelated eager work
    # between replays; every replay must reproduce the eager outputs and
    # gradients
    from rwkv7m_amd.screening import ScreenState
    wopt = WRITE if phase == "read_write" else {}
    case = _case(2, 40, 64, 80, 32, 80, 5, seed=31, use_age_mask=True,
                 **wopt)
    print(f"case: screening graph replay {phase}", flush=True)
    x, h, slots, ages, usage, P, cfg = case
    mod = _module(P, cfg, torch.float32)
    xd = torch.tensor(x, dtype=torch.float32, device="cuda",
                      requires_grad=True)
    hd = torch.tensor(h, dtype=torch.float32, device="cuda",
                      requires_grad=True)
    st = ScreenState(*(torch.tensor(a, dtype=torch.float32, device="cuda")
                       for a in (slots, ages, usage)))
    dh = torch.randn(xd.shape, device="cuda")
    params = list(mod.parameters())

    def clear():
        mod.zero_grad(set_to_none=True)
        xd.grad = None
        hd.grad = None

    def step():
        out, new, stats = mod(xd, hd, st, phase=phase)
        (out * dh).sum().backward()
        return [out, new.slots, new.usage_ema, stats["rel_read_mean"],
                stats["slot_usage_ema_mean"]]

    clear()
    ref = [t.detach().clone() for t in step()]
    ref_g = [p.grad.clone() for p in params] + [xd.grad.clone(),
                                                hd.grad.clone()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            clear()
            step()
    torch.cuda.current_stream().wait_stream(side)
    clear()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    grads = [p.grad for p in params] + [xd.grad, hd.grad]
    for i in range(3):
        noise = torch.randn(4096, device="cuda")
        (noise * noise).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs, ref)):
            torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6,
                                       msg=f"replay {i} output {k}")
        for k, (a, b) in enumerate(zip(grads, ref_g)):
            torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6,
                                       msg=f"replay {i} gradient {k}")


WRITE = dict(use_write_screening=True, write_rel_floor=0.05)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("opt", [dict(), dict(use_age_mask=True)], ids=str)
def test_write_phase_forward_matches_oracle(hip_lib, opt, dtype):
    case = _case(2, 29, 64, 80, 32, 80, 5, seed=51, **WRITE, **opt)
    _check_write_forward(case, dtype, f"screening read_write fwd {opt} {dtype}")


def _check_write_forward(case, dtype, name):
    print("case:", name, flush=True)
    _, _, _, _, out, new, stats = _run(case, dtype, phase="read_write")
    torch.cuda.synchronize()
    x, h, slots, ages, usage, P, cfg = case
    eh, (es, ea, eu), est = so.read_forward(_rnd(x, dtype), _rnd(h, dtype),
                                            slots, ages, usage, P, cfg,
                                            phase="read_write")
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for n, g, w in (("h", out, eh), ("slots_T", new.slots, es),
                    ("usage_T", new.usage_ema, eu)):
        e = _err(g, w)
        assert e <= tol, f"{name} {n}: {e:.3e} > {tol}"
    if dtype == torch.float32:
        assert torch.equal(new.ages.cpu(), torch.tensor(ea,
                                                        dtype=torch.float32))
    assert est["rel_write_mean"] > 0.0
    for k in so.STAT_NAMES:
        g, w = float(stats[k]), est[k]
        assert abs(g - w) <= tol * max(1.0, abs(w)), f"{name} stat {k}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("opt", [dict(), dict(use_age_mask=True)], ids=str)
def test_write_phase_backward_matches_autograd_oracle(hip_lib, opt, dtype):
    case = _case(2, 17, 64, 80, 32, 80, 5, seed=61, **WRITE, **opt)
    _check_write_backward(case, f"screening read_write bwd {opt} {dtype}",
                          dtype)


# The write kernels stage min(32, 2048 // max(d_slot, d_k)) steps at a
# time: these shapes cross several chunk boundaries.  d_slot 128, d_k 64:
# chunks of 16, weights in registers.  d_slot 300, d_k 30: chunks of 6,
# five channels per lane, weights in LDS, d_k not a multiple of 4.
# d_slot 260, d_k 72: chunks of 7, weights read from global memory, two key
# columns per lane.  d_slot 256, d_k 64 (the presets' sizes): chunks of 8,
# weights in LDS.
WRITE_CHUNKED = [(1, 70, 64, 128, 64, 64, 3), (1, 30, 48, 300, 30, 40, 2),
                 (1, 20, 48, 260, 72, 40, 2), (1, 20, 64, 256, 64, 64, 3)]


@pytest.mark.parametrize("shape", WRITE_CHUNKED, ids=str)
def test_write_phase_chunked(hip_lib, shape):
    case = _case(*shape, seed=71, **WRITE, use_age_mask=True)
    for dtype in (torch.float32, torch.bfloat16):
        _check_write_forward(case, dtype,
                             f"screening read_write fwd {shape} {dtype}")
        _check_write_backward(case, f"screening read_write bwd {shape} "
                              f"{dtype}", dtype)


def _check_write_backward(case, name, dtype=torch.float32):
    _check_backward(case, name, dtype, phase="read_write")
