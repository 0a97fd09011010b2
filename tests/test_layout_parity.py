"""GPU parity of the batch-major ([B, T, H, N]) entry points.

The reference's model holds its activations batch-major and swaps the first
two axes before and after every WKV call
(src/rwkv7m/model/nnx_model.py:695-698 and :709-711).  The ``_bthn`` entry
points read and write batch-major vectors in place of those two transposes.
Each head's arithmetic does not depend on where its vectors sit in HBM, so
the batch-major results must be bit-identical to the time-major results on
the transposed tensors, on every kernel path: the chunked MFMA kernels
(including their exact sequential fallback for strong decay and a partial
last chunk), the sequential kernels (fp32, other head sizes, other
intervals) and the single-token kernel.  One case per path is also checked
against the float64 oracle at the contract tolerance (2e-2 of max|oracle|
for bf16, 1e-4 for fp32).
"""

import numpy as np
import pytest
import torch

import oracle
from rwkv7m_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")
GRAD_NAMES = ("dr", "dw", "dk", "dv", "dneg_kk", "dkka", "ds0")


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _bt(t):
    """[T, B, ...] <-> [B, T, ...], contiguous."""
    return t.transpose(0, 1).contiguous()


def _both_layouts(hip, inp, ci):
    """Run forward, forward_with_aux and backward in both layouts; return
    the time-major results and the batch-major ones moved to time-major."""
    dev = {k: v.cuda() for k, v in inp.items()}
    tm = [dev[n] for n in NAMES]
    bm = [_bt(x) for x in tm]
    s0, dy, ds_t = dev["s0"], dev["dy"], dev["ds_t"]

    y_t, st_t = hip.forward(*tm, s0)
    y_b, st_b = hip.forward(*bm, s0, layout="bthn")
    (ya_t, sa_t), aux_t = hip.forward_with_aux(*tm, s0,
                                               checkpoint_interval=ci)
    (ya_b, sa_b), aux_b = hip.forward_with_aux(*bm, s0,
                                               checkpoint_interval=ci,
                                               layout="bthn")
    g_t = hip.backward(*tm, s0, dy, ds_t, *aux_t)
    g_b = hip.backward(*bm, s0, _bt(dy), ds_t, *aux_b, layout="bthn")
    torch.cuda.synchronize()
    assert y_b.shape == bm[0].shape and ya_b.shape == bm[0].shape
    time_major = {"y": y_t, "s_t": st_t, "y_aux": ya_t, "s_t_aux": sa_t,
                  "checkpoints": aux_t[0]}
    batch_major = {"y": _bt(y_b), "s_t": st_b, "y_aux": _bt(ya_b),
                   "s_t_aux": sa_b, "checkpoints": aux_b[0]}
    for name, gt, gb in zip(GRAD_NAMES, g_t, g_b):
        time_major[name] = gt
        batch_major[name] = gb if name == "ds0" else _bt(gb)
    return time_major, batch_major


def _assert_identical(time_major, batch_major, case):
    for name, want in time_major.items():
        got = batch_major[name]
        assert got.dtype == want.dtype and got.shape == want.shape, \
            f"{case} {name}: {got.dtype}{tuple(got.shape)} vs " \
            f"{want.dtype}{tuple(want.shape)}"
        if not torch.equal(got, want):
            diff = (got.float() - want.float()).abs().max().item()
            raise AssertionError(f"{case} {name}: batch-major differs from "
                                 f"time-major by {diff:.3e}")


def _check_oracle(results, inp, ci, tol, case):
    host = [_np(inp[n]) for n in NAMES]
    ey, es, _ = oracle.forward(*host, _np(inp["s0"]), checkpoint_interval=ci,
                               threads=8)
    egr = oracle.backward(*host, _np(inp["s0"]), _np(inp["dy"]),
                          _np(inp["ds_t"]), threads=8)
    expected = dict(zip(GRAD_NAMES, egr), y=ey, s_t=es)
    for name, e in expected.items():
        err = oracle.normalized_max_error(_np(results[name]), e)
        assert err <= tol, f"{case} {name}: {err:.3e} > {tol}"


@pytest.mark.parametrize("ci", [16, 32])
@pytest.mark.parametrize("T", [2, 45, 96])
def test_chunked_batch_major_equals_time_major(hip, T, ci):
    case = f"chunked bthn T{T} B3 H2 N64 L{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(T, 3, 2, 64, seed=300 + T + ci, state_std=0.1,
                      dstate_std=0.1)
    tm, bm = _both_layouts(hip, inp, ci)
    assert tm["checkpoints"].dtype == torch.bfloat16  # the MFMA path
    _assert_identical(tm, bm, case)
    if T == 45:
        _check_oracle(bm, inp, ci, 2e-2, case)


def test_chunked_batch_major_mixed_fallback(hip):
    # strong decay in tokens 32..63 of batch 1 only: those chunks take the
    # exact sequential fallback inside the chunked kernels
    case = "chunked bthn mixed decay T100 B2 H2 L32"
    print("case:", case, flush=True)
    inp = make_inputs(100, 2, 2, 64, seed=71, state_std=0.1, dstate_std=0.1)
    w = inp["w"].float()
    w[32:64, 1] += 3.0
    inp["w"] = w.to(torch.bfloat16)
    tm, bm = _both_layouts(hip, inp, 32)
    _assert_identical(tm, bm, case)
    _check_oracle(bm, inp, 32, 2e-2, case)


@pytest.mark.parametrize("dtype,N,ci", [
    (torch.float32, 64, 16),
    (torch.float32, 8, 5),
    (torch.bfloat16, 32, 16),
    (torch.bfloat16, 64, 3),
    (torch.bfloat16, 128, 16),
    (torch.float32, 128, 7),
])
def test_sequential_batch_major_equals_time_major(hip, dtype, N, ci):
    case = f"sequential bthn T37 B2 H3 N{N} {dtype} ci{ci}"
    print("case:", case, flush=True)
    inp = make_inputs(37, 2, 3, N, dtype=dtype, seed=17 + N + ci,
                      state_std=0.1, dstate_std=0.1)
    tm, bm = _both_layouts(hip, inp, ci)
    _assert_identical(tm, bm, case)
    if dtype == torch.float32 and N in (64, 128):
        _check_oracle(bm, inp, ci, 1e-4, case)


def test_single_token_batch_major(hip):
    # T = 1: [1, B, H, N] and [B, 1, H, N] are the same memory, and both
    # calls reach the single-token kernel
    case = "bthn T1 B4 H3 N64"
    print("case:", case, flush=True)
    inp = make_inputs(1, 4, 3, 64, seed=5, state_std=0.5)
    dev = {k: v.cuda() for k, v in inp.items()}
    tm = [dev[n] for n in NAMES]
    y_t, s_t = hip.forward(*tm, dev["s0"])
    y_b, s_b = hip.forward(*(_bt(x) for x in tm), dev["s0"], layout="bthn")
    torch.cuda.synchronize()
    assert torch.equal(_bt(y_b), y_t) and torch.equal(s_b, s_t)


def test_layout_argument_is_checked(hip):
    inp = make_inputs(4, 1, 1, 64, seed=1)
    dev = [inp[n].cuda() for n in NAMES]
    with pytest.raises(ValueError, match="layout"):
        hip.forward(*dev, inp["s0"].cuda(), layout="bhtn")


def test_operator_batch_major_through_hip_backend(hip):
    # wkv7_batch_major with the HIP backend registered: forward and autograd
    # backward on the batch-major tensors equal the time-major operator on
    # the transposed ones
    from rwkv7m_amd.kernels.wkv_ffi import unregister_wkv_ffi_backend
    from rwkv7m_amd.wkv import wkv7, wkv7_batch_major
    case = "operator bthn T70 B2 H2 N64"
    print("case:", case, flush=True)
    inp = make_inputs(70, 2, 2, 64, seed=23, state_std=0.1)
    unregister_wkv_ffi_backend()
    hip.register_hip_backend()
    try:
        tm = [inp[n].cuda().requires_grad_(True) for n in NAMES]
        s0 = inp["s0"].cuda().requires_grad_(True)
        bm = [_bt(x.detach()).requires_grad_(True) for x in tm]
        s0b = s0.detach().clone().requires_grad_(True)
        y_t, st_t = wkv7(*tm, s0, "ffi")
        y_b, st_b = wkv7_batch_major(*bm, s0b, "ffi")
        dy = inp["dy"].cuda()
        g_t = torch.autograd.grad((y_t.float() * dy.float()).sum()
                                  + st_t.sum(), tm + [s0])
        g_b = torch.autograd.grad((y_b.float() * _bt(dy).float()).sum()
                                  + st_b.sum(), bm + [s0b])
        torch.cuda.synchronize()
        assert torch.equal(_bt(y_b), y_t) and torch.equal(st_b, st_t)
        for name, a, b in zip(GRAD_NAMES, g_t, g_b):
            want = a if name == "ds0" else _bt(a)
            assert torch.equal(b, want), f"{case} {name}"
    finally:
        unregister_wkv_ffi_backend()
