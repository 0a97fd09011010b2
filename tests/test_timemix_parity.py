"""GPU parity of the fused time-mix producers and consumer
(``rwkv7m_timemix_*``, include/rwkv7m_timemix.h) against the float64 oracle
(oracle/timemix_oracle.py, restating nnx_model.py:630, :683-694, :709-727).

Tolerances (the contract's): normalised max error (max |got - want| over
max |want|) <= 2e-2 for bf16 activations and <= 1e-4 for fp32, on every
output and every parameter gradient.  The oracle runs on the same
(dtype-rounded) inputs.

Shapes cover every launch geometry: several rows per block (C < 2048, with
and without idle threads), one row per block (C = 2048), two column tiles
with a partial second one (C = 3072), every head size (8 ... 128), one row,
no rows, and enough rows for each thread to stride several times.  At the
headline shape (B=8, T=4096, C=2048) sampled rows are checked against the
oracle (every output is row-local) and the parameter gradients through
additivity over row halves.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import timemix_oracle as tmo

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}
SHAPES = [(1, 1, 64), (37, 3, 64), (64, 32, 64), (50, 48, 64), (45, 12, 64),
          (33, 4, 8), (20, 5, 16), (19, 3, 32), (17, 2, 128)]


@pytest.fixture(scope="module")
def tm(hip_lib):
    from rwkv7m_amd.kernels import timemix_hip
    return timemix_hip


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _err(got, want):
    return oracle.normalized_max_error(_f64(got), want)


def _make(rows, H, N, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    C = H * N

    def act(scale=1.0, shift=0.0):
        return (torch.randn(rows, C, generator=g) * scale + shift).to(dtype)

    a = {"w_raw": act(2.0, -1.0), "k": act(), "a": torch.sigmoid(
        torch.randn(rows, C, generator=g)).to(dtype),
        "y": act(0.7, 0.3), "r": act(), "v": act(), "g": act()}
    a.update({f"d{i}": act() for i in range(6)})
    p = {"k_k": 0.7 + 0.1 * torch.randn(C, generator=g),
         "k_a": 1.0 + 0.05 * torch.randn(C, generator=g),
         "r_k": -0.04 + 0.3 * torch.randn(C, generator=g),
         "scale": 0.5 + torch.rand(C, generator=g),
         "bias": 0.2 * torch.randn(C, generator=g)}
    return a, p


def _check(name, got, want, tol, case):
    e = _err(got, want)
    assert e <= tol, f"{case} {name}: normalized error {e:.3e} > {tol}"


def _run_inputs(tm, a, p, N, dk2=False):
    dev = {k: v.cuda() for k, v in {**a, **p}.items()}
    fwd = tm.inputs_forward(dev["w_raw"], dev["k"], dev["a"], dev["k_k"],
                            dev["k_a"], N)
    bwd = tm.inputs_backward(dev["w_raw"], dev["k"], dev["a"], dev["k_k"],
                             dev["k_a"], dev["d0"], dev["d1"], dev["d2"],
                             dev["d3"], N,
                             dk_out2=dev["d4"] if dk2 else None)
    torch.cuda.synchronize()
    return fwd, bwd


def _run_output(tm, a, p, N):
    dev = {k: v.cuda() for k, v in {**a, **p}.items()}
    args = [dev[n] for n in ("y", "r", "k", "v", "g", "r_k", "scale",
                             "bias")]
    out = tm.output_forward(*args, N)
    bwd = tm.output_backward(*args, dev["d5"], N)
    torch.cuda.synchronize()
    return out, bwd


def _oracle_inputs(a, p, N, dk2=False):
    h = {k: _f64(v) for k, v in {**a, **p}.items()}
    fwd = tmo.wkv_inputs(h["w_raw"], h["k"], h["a"], h["k_k"], h["k_a"], N)
    dkp = h["d1"] + h["d4"] if dk2 else h["d1"]
    bwd = tmo.wkv_inputs_backward(h["w_raw"], h["k"], h["a"], h["k_k"],
                                  h["k_a"], h["d0"], dkp, h["d2"], h["d3"],
                                  N)
    return fwd, bwd


def _oracle_output(a, p, N):
    h = {k: _f64(v) for k, v in {**a, **p}.items()}
    args = [h[n] for n in ("y", "r", "k", "v", "g", "r_k", "scale", "bias")]
    return (tmo.wkv_output(*args, N),
            tmo.wkv_output_backward(*args, h["d5"], N))


IN_NAMES = ("w", "k_out", "neg_kk", "kka")
IN_GRADS = ("dw_raw", "dk", "da", "dk_k", "dk_a")
OUT_GRADS = ("dy", "dr", "dk", "dv", "dg", "dr_k", "dln_scale", "dln_bias")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_inputs_match_oracle(tm, rows, H, N, dtype):
    case = f"inputs rows{rows} H{H} N{N} {dtype}"
    print("case:", case, flush=True)
    a, p = _make(rows, H, N, dtype, seed=rows * 7 + H + N)
    fwd, bwd = _run_inputs(tm, a, p, N, dk2=(rows % 2 == 1))
    efwd, ebwd = _oracle_inputs(a, p, N, dk2=(rows % 2 == 1))
    for name, g_, w_ in zip(IN_NAMES + IN_GRADS, (*fwd, *bwd),
                            (*efwd, *ebwd)):
        assert g_.dtype == (torch.float32 if name in ("dk_k", "dk_a")
                            else dtype)
        _check(name, g_, w_, TOL[dtype], case)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,H,N", SHAPES)
def test_output_matches_oracle(tm, rows, H, N, dtype):
    case = f"output rows{rows} H{H} N{N} {dtype}"
    print("case:", case, flush=True)
    a, p = _make(rows, H, N, dtype, seed=rows * 11 + H + N)
    out, bwd = _run_output(tm, a, p, N)
    eout, ebwd = _oracle_output(a, p, N)
    _check("out", out, eout, TOL[dtype], case)
    for name, g_, w_ in zip(OUT_GRADS, bwd, ebwd):
        _check(name, g_, w_, TOL[dtype], case)


def test_many_rows_per_thread(tm):
    # 40000 rows of C = 128: each thread strides over several rows in both
    # directions (16 rows per block, at most 2048 / 1024 blocks)
    case = "rows40000 H2 N64 bf16"
    print("case:", case, flush=True)
    a, p = _make(40000, 2, 64, torch.bfloat16, seed=9)
    fwd, bwd = _run_inputs(tm, a, p, 64)
    efwd, ebwd = _oracle_inputs(a, p, 64)
    for name, g_, w_ in zip(IN_NAMES + IN_GRADS, (*fwd, *bwd),
                            (*efwd, *ebwd)):
        _check(name, g_, w_, 2e-2, case)
    out, obwd = _run_output(tm, a, p, 64)
    eout, eobwd = _oracle_output(a, p, 64)
    _check("out", out, eout, 2e-2, case)
    for name, g_, w_ in zip(OUT_GRADS, obwd, eobwd):
        _check(name, g_, w_, 2e-2, case)


def test_no_rows_gives_empty_outputs_and_zero_parameter_gradients(tm):
    a, p = _make(0, 3, 64, torch.bfloat16, seed=1)
    fwd, bwd = _run_inputs(tm, a, p, 64)
    assert all(x.numel() == 0 for x in fwd + bwd[:3])
    assert all(torch.equal(x, torch.zeros(192, device="cuda"))
               for x in bwd[3:])
    out, obwd = _run_output(tm, a, p, 64)
    assert out.numel() == 0
    assert all(torch.equal(x, torch.zeros(192, device="cuda"))
               for x in obwd[5:])


def test_backward_is_deterministic_and_dk2_equals_presummed(tm):
    a, p = _make(300, 32, 64, torch.float32, seed=3)
    _, b1 = _run_inputs(tm, a, p, 64, dk2=True)
    _, b2 = _run_inputs(tm, a, p, 64, dk2=True)
    for x, y in zip(b1, b2):
        assert torch.equal(x, y)
    a2 = dict(a)
    a2["d1"] = a["d1"] + a["d4"]
    _, b3 = _run_inputs(tm, a2, p, 64)
    for x, y in zip(b1, b3):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-5)
    _, o1 = _run_output(tm, a, p, 64)
    _, o2 = _run_output(tm, a, p, 64)
    for x, y in zip(o1, o2):
        assert torch.equal(x, y)


def test_unaligned_views_are_served(tm):
    # a view starting one element into its storage is not 16-byte aligned;
    # the wrapper hands the kernels an aligned copy
    a, p = _make(9, 2, 64, torch.bfloat16, seed=4)
    dev = {k: v.cuda() for k, v in {**a, **p}.items()}
    base = torch.empty(9 * 128 + 1, dtype=torch.bfloat16, device="cuda")
    view = base[1:].view(9, 128)
    view.copy_(dev["w_raw"])
    assert view.data_ptr() % 16
    got = tm.inputs_forward(view, dev["k"], dev["a"], dev["k_k"],
                            dev["k_a"], 64)
    want = tm.inputs_forward(dev["w_raw"], dev["k"], dev["a"], dev["k_k"],
                             dev["k_a"], 64)
    for x, y in zip(got, want):
        assert torch.equal(x, y)


def test_headline_shape_sampled_rows_and_additivity(tm):
    # B=8, T=4096, H=32, N=64: outputs are row-local, so sampled rows are
    # checked against the oracle exactly as at small sizes; the parameter
    # gradients (sums over all rows) must equal the sums of the gradients
    # of the two row halves
    rows, H, N = 8 * 4096, 32, 64
    case = "headline rows32768 H32 N64 bf16"
    print("case:", case, flush=True)
    a, p = _make(rows, H, N, torch.bfloat16, seed=5)
    fwd, bwd = _run_inputs(tm, a, p, N)
    out, obwd = _run_output(tm, a, p, N)
    idx = torch.randperm(rows, generator=torch.Generator().manual_seed(6)
                         )[:96]
    sa = {k: v[idx] for k, v in a.items()}
    efwd, ebwd = _oracle_inputs(sa, p, N)
    eout, eobwd = _oracle_output(sa, p, N)
    for name, g_, w_ in zip(IN_NAMES + IN_GRADS[:3], (*fwd, *bwd[:3]),
                            (*efwd, *ebwd[:3])):
        _check(name, g_[idx.cuda()], w_, 2e-2, case)
    _check("out", out[idx.cuda()], eout, 2e-2, case)
    for name, g_, w_ in zip(OUT_GRADS[:5], obwd[:5], eobwd[:5]):
        _check(name, g_[idx.cuda()], w_, 2e-2, case)
    half = rows // 2
    lo = {k: v[:half] for k, v in a.items()}
    hi = {k: v[half:] for k, v in a.items()}
    _, blo = _run_inputs(tm, lo, p, N)
    _, bhi = _run_inputs(tm, hi, p, N)
    _, olo = _run_output(tm, lo, p, N)
    _, ohi = _run_output(tm, hi, p, N)
    for full, x, y in zip(bwd[3:] + obwd[5:], blo[3:] + olo[5:],
                          bhi[3:] + ohi[5:]):
        s = (x.double() + y.double())
        e = (full.double() - s).abs().max().item() / s.abs().max().item()
        assert e <= 1e-5, f"{case} parameter gradient additivity {e:.3e}"


# ---------------------------------------------------------------------------
# The fused time-mix WKV section against the oracle chain
# ---------------------------------------------------------------------------

def _chain_oracle(a, p, s0, dout, ds_t, B, T, H, N, bf16):
    """Oracle chain with the reference's bf16 materialisations (w, k',
    neg_kk, kka and y are bf16 arrays in the reference's model)."""
    rnd = oracle.bf16_round if bf16 else (lambda x: x)
    h = {k: _f64(v) for k, v in {**a, **p}.items()}
    C = H * N
    w, kp, nkk, kka = (rnd(x) for x in tmo.wkv_inputs(
        h["w_raw"], h["k"], h["a"], h["k_k"], h["k_a"], N))

    def tm_(x):  # [B*T, C] -> time-major [T, B, H, N]
        return x.reshape(B, T, H, N).transpose(1, 0, 2, 3)

    def bm(x):  # time-major -> [B*T, C]
        return x.transpose(1, 0, 2, 3).reshape(B * T, C)

    vecs = [tm_(x) for x in (h["r"], w, kp, h["v"], nkk, kka)]
    y, s_t = oracle.forward(*vecs, s0, threads=8)
    y = rnd(bm(y))
    args = (y, h["r"], kp, h["v"], h["g"], h["r_k"], h["scale"], h["bias"])
    out = tmo.wkv_output(*args, N)
    dy, dr_c, dk_c, dv_c, dg, drk, dsc, dbi = tmo.wkv_output_backward(
        *args, dout, N)
    gr = oracle.backward(*vecs, s0, tm_(rnd(dy)), ds_t, threads=8)
    dr, dw, dk_w, dv, dnkk, dkka, ds0 = gr
    dx, dk, da, dkk_p, dka_p = tmo.wkv_inputs_backward(
        h["w_raw"], h["k"], h["a"], h["k_k"], h["k_a"], bm(dw),
        bm(dk_w) + dk_c, bm(dnkk), bm(dkka), N)
    grads = {"r": bm(dr) + dr_c, "w_raw": dx, "k": dk, "v": bm(dv) + dv_c,
             "a": da, "g": dg, "k_k": dkk_p, "k_a": dka_p, "r_k": drk,
             "scale": dsc, "bias": dbi, "s0": ds0}
    return out, s_t, grads


@pytest.mark.parametrize("dtype,T,H,N", [(torch.bfloat16, 45, 2, 64),
                                         (torch.bfloat16, 70, 3, 64),
                                         (torch.float32, 23, 2, 16)])
def test_time_mix_wkv_matches_oracle_chain(hip_lib, dtype, T, H, N):
    from rwkv7m_amd.timemix import time_mix_wkv
    B = 2
    case = f"time_mix_wkv B{B} T{T} H{H} N{N} {dtype}"
    print("case:", case, flush=True)
    a, p = _make(B * T, H, N, dtype, seed=T + N)
    a["w_raw"] = (a["w_raw"].float() * 0.5 - 0.5).to(dtype)
    g = torch.Generator().manual_seed(T)
    s0 = torch.randn(B, H, N, N, generator=g) * 0.1
    dout = torch.randn(B, T, H * N, generator=g).to(dtype)
    ds_t = torch.randn(B, H, N, N, generator=g) * 0.1
    names = ("r", "w_raw", "k", "v", "a", "g")
    leaves = {n: a[n].view(B, T, H * N).cuda().requires_grad_(True)
              for n in names}
    pl = {"k_k": p["k_k"].view(1, 1, -1), "k_a": p["k_a"].view(1, 1, -1),
          "r_k": p["r_k"].view(H, N), "scale": p["scale"],
          "bias": p["bias"]}
    pl = {k: v.cuda().requires_grad_(True) for k, v in pl.items()}
    s0d = s0.cuda().requires_grad_(True)
    out, s_t = time_mix_wkv(*(leaves[n] for n in names), pl["k_k"],
                            pl["k_a"], pl["r_k"], pl["scale"], pl["bias"],
                            s0d, n_heads=H)
    loss = (out.float() * dout.cuda().float()).sum() + \
        (s_t * ds_t.cuda()).sum()
    loss.backward()
    torch.cuda.synchronize()
    eout, es_t, eg = _chain_oracle(a, p, s0.double().numpy(),
                                   _f64(dout).reshape(B * T, -1),
                                   ds_t.double().numpy(), B, T, H, N,
                                   dtype == torch.bfloat16)
    tol = TOL[dtype]
    _check("out", out.reshape(B * T, -1), eout, tol, case)
    _check("s_t", s_t, es_t, tol, case)
    for n in names:
        _check("d" + n, leaves[n].grad.reshape(B * T, -1), eg[n], tol, case)
    for n in pl:
        assert pl[n].grad.shape == pl[n].shape
        _check("d" + n, pl[n].grad.reshape(-1), eg[n], tol, case)
    _check("ds0", s0d.grad, eg["s0"], tol, case)


def test_time_mix_wkv_equals_separate_ops(hip_lib):
    # producers, batch-major WKV and consumer as three autograd ops give the
    # fused section's results (the fused backward adds the consumer's
    # cotangents of r, k' and v in fp32 inside the WKV backward, the
    # separate ops in bf16)
    import rwkv7m_amd
    from rwkv7m_amd.kernels.wkv_ffi import unregister_wkv_ffi_backend
    from rwkv7m_amd.timemix import time_mix_wkv, wkv7_inputs, wkv7_output
    B, T, H, N = 2, 40, 2, 64
    a, p = _make(B * T, H, N, torch.bfloat16, seed=12)
    names = ("r", "w_raw", "k", "v", "a", "g")
    dout = torch.randn(B, T, H * N).to(torch.bfloat16).cuda()
    results = []
    unregister_wkv_ffi_backend()
    rwkv7m_amd.register_hip_backend()
    try:
        for fused in (True, False):
            lv = {n: a[n].view(B, T, -1).cuda().requires_grad_(True)
                  for n in names}
            pv = {k: v.cuda().requires_grad_(True) for k, v in p.items()}
            s0 = torch.zeros(B, H, N, N, device="cuda", requires_grad=True)
            if fused:
                out, s_t = time_mix_wkv(
                    *(lv[n] for n in names), pv["k_k"], pv["k_a"],
                    pv["r_k"], pv["scale"], pv["bias"], s0, n_heads=H)
            else:
                w, kp, nkk, kka = wkv7_inputs(lv["w_raw"], lv["k"], lv["a"],
                                              pv["k_k"], pv["k_a"], H)
                r_h = lv["r"].view(B, T, H, N)
                v_h = lv["v"].view(B, T, H, N)
                y, s_t = rwkv7m_amd.wkv7_batch_major(r_h, w, kp, v_h, nkk,
                                                     kka, s0, "ffi")
                out = wkv7_output(y, r_h, kp, v_h, lv["g"], pv["r_k"],
                                  pv["scale"], pv["bias"])
            ((out.float() * dout.float()).sum() + s_t.sum()).backward()
            results.append([out, s_t] + [lv[n].grad for n in names] +
                           [pv[n].grad for n in p] + [s0.grad])
    finally:
        unregister_wkv_ffi_backend()
    torch.cuda.synchronize()
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])
    for x, y in zip(results[0][2:], results[1][2:]):
        e = oracle.normalized_max_error(_f64(x), _f64(y))
        assert e <= 1e-2, e
