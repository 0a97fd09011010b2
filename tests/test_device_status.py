"""The MFMA kernels' bounded hand-over waits fail loudly, never silently.

The wave-specialised forward hands each chunk from producer waves to chain
waves through LDS, the backward between chain and worker waves, and every
wait for a hand-over polls a bounded number of times.  Here the host shrinks
that bound to one poll (rwkv7m_debug_set_wait_limit), so the waiting waves
give up before the hand-over arrives.  Every kernel still exits normally (all accesses stay in bounds);
the call must then return NaN in every output of the affected heads, and
rwkv7m_device_status must report the failures.  With the default bound
restored, the same call matches the oracle and the status is clean.
"""

import numpy as np
import pytest
import torch

import oracle
from rwkv7m_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def test_forward_wait_that_gives_up_poisons_outputs_and_reports(hip):
    print("case: wave forward with a one-poll wait budget", flush=True)
    inp = make_inputs(256, 2, 2, 64, seed=61, state_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    hip.device_status()  # start from a clean count
    hip.set_wait_limit(1)
    try:
        (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                             checkpoint_interval=32)
        assert hip.last_path() == "wave_forward"
        torch.cuda.synchronize()
    finally:
        hip.set_wait_limit(0)
    with pytest.raises(RuntimeError, match="bounded wait"):
        hip.device_status()
    # the status call cleared the count
    hip.device_status()
    # every output of a failed head is NaN; a head whose waits all happened
    # to succeed must be exact, so no head may hold silent garbage
    ey, es = oracle.forward(*[_np(inp[n]) for n in NAMES], _np(inp["s0"]))
    failed = 0
    for b in range(2):
        for h in range(2):
            yh, sh, ck = y[:, b, h], s_t[b, h], aux[0][:, b, h]
            if torch.isnan(sh).all():
                failed += 1
                assert torch.isnan(yh.float()).all()
                assert torch.isnan(ck.float()).all()
            else:
                assert torch.isfinite(yh.float()).all()
                err = oracle.normalized_max_error(_np(yh), ey[:, b, h])
                assert err <= 2e-2
    assert failed >= 1

    # default budget: clean and correct
    (y, s_t), _ = hip.forward_with_aux(*vecs, dev["s0"],
                                       checkpoint_interval=32)
    torch.cuda.synchronize()
    hip.device_status()
    assert oracle.normalized_max_error(_np(y), ey) <= 2e-2
    assert oracle.normalized_max_error(_np(s_t), es) <= 2e-2


def test_backward_wait_that_gives_up_poisons_outputs_and_reports(hip):
    # the wave backward hands chunks between chain and worker waves the
    # same way; with a one-poll budget its waits give up before the
    # hand-overs arrive
    print("case: wave backward with a one-poll wait budget", flush=True)
    T, B, H = 256, 2, 2
    inp = make_inputs(T, B, H, 64, seed=62, state_std=0.1, dstate_std=0.1)
    dev = {k: v.cuda() for k, v in inp.items()}
    vecs = [dev[n] for n in NAMES]
    (y, s_t), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                         checkpoint_interval=16)
    torch.cuda.synchronize()
    hip.device_status()
    hip.set_wait_limit(1)
    try:
        grads = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux)
        assert hip.last_path() == "wave_backward"
        torch.cuda.synchronize()
    finally:
        hip.set_wait_limit(0)
    with pytest.raises(RuntimeError, match="bounded wait"):
        hip.device_status()
    hip.device_status()
    host = [_np(inp[n]) for n in NAMES]
    egr = oracle.backward(*host, _np(inp["s0"]), _np(inp["dy"]),
                          _np(inp["ds_t"]))
    failed = 0
    for b in range(B):
        for h in range(H):
            gh = [g[:, b, h] for g in grads[:6]] + [grads[6][b, h]]
            if torch.isnan(gh[6]).all():
                failed += 1
                for g in gh:
                    assert torch.isnan(g.float()).all()
            else:
                ehs = [e[:, b, h] for e in egr[:6]] + [egr[6][b, h]]
                for g, e in zip(gh, ehs):
                    assert torch.isfinite(g.float()).all()
                    assert oracle.normalized_max_error(_np(g), e) <= 2e-2
    assert failed >= 1

    # default budget: clean and correct
    grads = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux)
    torch.cuda.synchronize()
    hip.device_status()
    for g, e in zip(grads, egr):
        assert oracle.normalized_max_error(_np(g), e) <= 2e-2
