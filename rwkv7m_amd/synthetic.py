"""Synthetic WKV-7 inputs with the distributions of the model's own producer.

The model builds the WKV inputs at src/rwkv7m/model/nnx_model.py:630 and
:683-694: ``w = -softplus(-x) - 0.5`` (so the decay ``exp(-exp(w))`` equals
``exp(-0.6065 * sigmoid(x))``), ``kk`` L2-normalised per head,
``neg_kk = -kk`` and ``kka = kk * a`` with ``a = sigmoid(.)`` in (0, 1).

Draw order: x_r, x_k, x_v, x_w, z_kk, x_a, S0, dy, dS_T.  ``generator``
"numpy" uses PCG64 on the host (reproducible, for parity tests and golden
fixtures); "torch" draws on the target device (fast, for full-size benches).
"""

from __future__ import annotations

import numpy as np
import torch

FIELDS = ("r", "w", "k", "v", "neg_kk", "kka", "s0", "dy", "ds_t")


def _softplus(x):
    return np.logaddexp(0.0, x)


def make_inputs(T: int, B: int, H: int, N: int, *, dtype=torch.bfloat16,
                seed: int = 0, slow_decay: bool = False,
                state_std: float = 0.0, dstate_std: float = 0.0,
                dy_std: float = 1.0, device="cpu",
                generator: str = "numpy") -> dict:
    """Return a dict of torch tensors: vectors ``[T,B,H,N]`` in ``dtype``,
    ``s0``/``ds_t`` ``[B,H,N,N]`` fp32, ``dy`` in ``dtype``."""
    vshape, sshape = (T, B, H, N), (B, H, N, N)
    w_mean = -2.0 if slow_decay else 0.0
    if generator == "numpy":
        rng = np.random.Generator(np.random.PCG64(seed))
        x_r, x_k, x_v = (rng.standard_normal(vshape) for _ in range(3))
        x_w = rng.standard_normal(vshape) + w_mean
        z = rng.standard_normal(vshape)
        x_a = rng.standard_normal(vshape)
        s0 = rng.standard_normal(sshape) * state_std
        dy = rng.standard_normal(vshape) * dy_std
        ds_t = rng.standard_normal(sshape) * dstate_std
        w = -_softplus(-x_w) - 0.5
        kk = z / np.maximum(np.linalg.norm(z, axis=-1, keepdims=True), 1e-12)
        kka = kk / (1.0 + np.exp(-x_a))
        out = {"r": x_r, "w": w, "k": x_k, "v": x_v, "neg_kk": -kk,
               "kka": kka, "s0": s0, "dy": dy, "ds_t": ds_t}
        res = {}
        for name, arr in out.items():
            t = torch.from_numpy(np.ascontiguousarray(arr, np.float32))
            if name not in ("s0", "ds_t"):
                t = t.to(dtype)
            res[name] = t.to(device)
        return res
    if generator != "torch":
        raise ValueError(f"unknown generator {generator!r}")
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def normal(shape, std=1.0, mean=0.0):
        x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        if std != 1.0:
            x.mul_(std)
        if mean != 0.0:
            x.add_(mean)
        return x

    res = {}
    res["r"] = normal(vshape).to(dtype)
    res["k"] = normal(vshape).to(dtype)
    res["v"] = normal(vshape).to(dtype)
    x_w = normal(vshape, mean=w_mean)
    res["w"] = (-torch.nn.functional.softplus(-x_w) - 0.5).to(dtype)
    del x_w
    z = normal(vshape)
    z = z / z.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    res["neg_kk"] = (-z).to(dtype)
    res["kka"] = (z * torch.sigmoid(normal(vshape))).to(dtype)
    del z
    res["s0"] = normal(sshape, std=state_std) if state_std else \
        torch.zeros(sshape, device=dev)
    res["dy"] = normal(vshape, std=dy_std).to(dtype)
    res["ds_t"] = normal(sshape, std=dstate_std) if dstate_std else \
        torch.zeros(sshape, device=dev)
    return {k: res[k] for k in FIELDS}


# The benchmark configurations (shapes, dtypes and distributions); state
# noise "N(0, 0.1)" is read as standard deviation 0.1.
CONFIGS = {
    0: dict(T=64, B=2, H=4, N=16, dtype=torch.float32, seed=1000),
    1: dict(T=512, B=8, H=12, N=64, dtype=torch.bfloat16, seed=1001),
    2: dict(T=4096, B=8, H=32, N=64, dtype=torch.bfloat16, seed=1002),
    3: dict(T=1, B=256, H=64, N=64, dtype=torch.bfloat16, seed=1003,
            state_std=0.1),
    4: dict(T=8192, B=4, H=64, N=64, dtype=torch.bfloat16, seed=1004,
            slow_decay=True, state_std=0.1,
            dstate_std=0.1),
}


def config_inputs(index: int, *, device="cpu", generator="numpy",
                  **overrides) -> dict:
    cfg = dict(CONFIGS[index])
    cfg.update(overrides)
    T, B, H, N = cfg.pop("T"), cfg.pop("B"), cfg.pop("H"), cfg.pop("N")
    return make_inputs(T, B, H, N, device=device, generator=generator,
                       **cfg)


__all__ = ["CONFIGS", "FIELDS", "config_inputs", "make_inputs"]
