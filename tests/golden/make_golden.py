"""Write the golden WKV-7 fixtures in this directory from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each fixture is an .npz holding the inputs (bf16 inputs as uint16 bit
patterns, fp32 ones as float32) and the float64 oracle's outputs stored as
float32: y (unrounded), s_t, and, where present, the seven cotangents for the
stored dy / ds_t. The reference's only JAX-free known answer
(tests/test_upstream_rwkv7_parity.py:265-297, rng 19, one step, n=4) is kept
as kat_step.npz with the reference test's own expected values.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from rwkv7m_amd.synthetic import config_inputs, make_inputs  # noqa: E402

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")


def _pack(inputs, bf16: bool):
    out = {}
    for name in (*NAMES, "dy"):
        x = inputs[name].float().numpy()
        out[name] = oracle.bf16_bits(x) if bf16 else x.astype(np.float32)
    out["s0"] = inputs["s0"].numpy().astype(np.float32)
    out["ds_t"] = inputs["ds_t"].numpy().astype(np.float32)
    out["is_bf16"] = np.array(bf16)
    return out


def _write(name, inputs, bf16, with_grads=True):
    vecs = [inputs[n].float().numpy().astype(np.float64) for n in NAMES]
    s0 = inputs["s0"].numpy().astype(np.float64)
    data = _pack(inputs, bf16)
    y, s_t = oracle.forward(*vecs, s0)
    data["y"] = y.astype(np.float32)
    data["s_t"] = s_t.astype(np.float32)
    if with_grads:
        dy = inputs["dy"].float().numpy().astype(np.float64)
        grads = oracle.backward(*vecs, s0, dy,
                                inputs["ds_t"].numpy().astype(np.float64))
        for gname, g in zip(("dr", "dw", "dk", "dv", "dneg_kk", "dkka",
                             "ds0"), grads):
            data[gname] = g.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, name), **data)
    print("wrote", name)


def kat_step():
    rng = np.random.default_rng(19)
    n = 4
    state = rng.normal(size=(1, 1, n, n)).astype(np.float32)
    r, raw_w, k, v, a, b = (rng.normal(size=(1, 1, n)).astype(np.float32)
                            for _ in range(6))
    decay = np.exp(-np.exp(raw_w))
    sa = np.einsum("bhij,bhj->bhi", state, a)
    s_t = (state * decay[..., None, :] + np.einsum("bhi,bhj->bhij", sa, b)
           + np.einsum("bhi,bhj->bhij", v, k))
    y = np.einsum("bhij,bhj->bhi", s_t, r)
    np.savez_compressed(
        os.path.join(HERE, "kat_step.npz"), r=r[None], w=raw_w[None],
        k=k[None], v=v[None], neg_kk=a[None], kka=b[None], s0=state,
        y=y[None], s_t=s_t, is_bf16=np.array(False))
    print("wrote kat_step.npz")


def main():
    kat_step()
    # benchmark configuration 0 (fp32 forward, tiny_config shape), full size.
    _write("config0_fwd.npz", config_inputs(0), bf16=False, with_grads=False)
    # small bf16 fwd+bwd with ragged T (not a multiple of any chunk length)
    _write("bf16_t37_n16.npz",
           make_inputs(37, 2, 3, 16, seed=2001, state_std=0.1,
                       dstate_std=0.1), bf16=True)
    # the training head size: bf16 fwd+bwd, N=64, zero S0 (configs 1-2 style)
    _write("bf16_t80_n64.npz", make_inputs(80, 1, 2, 64, seed=2002),
           bf16=True)
    # carry-state slow decay (config 4 style), nonzero S0 and dS_T
    _write("bf16_carry_slow_t96_n64.npz",
           make_inputs(96, 1, 2, 64, seed=2003, slow_decay=True,
                       state_std=0.1, dstate_std=0.1), bf16=True)
    # one decode step (config 3 style), nonzero S0
    _write("bf16_decode_n64.npz",
           make_inputs(1, 3, 2, 64, seed=2004, state_std=0.1), bf16=True)
    # fp32 fwd+bwd (reference unit-test scale, tests/test_wkv_api.py:9-18)
    import torch
    small = make_inputs(3, 1, 2, 4, seed=2005, dtype=torch.float32,
                        state_std=0.1, dstate_std=0.1)
    _write("f32_t3_n4.npz", small, bf16=False)


if __name__ == "__main__":
    main()
