"""HIP-graph capture of the WKV operator and the fused time-mix section
(GPU).  Serving loops and launch-bound training steps capture these calls;
every replay, with unrelated eager work between replays, must reproduce
the eager outputs and gradients.  The library records no memset nodes
(clears are fill kernels) and makes no host synchronisation inside a call.
"""

import pytest
import torch

from rwkv7m_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")


def _replay_check(step, leaves, case):
    def clear():
        for t in leaves:
            t.grad = None

    clear()
    ref = [t.detach().clone() for t in step()]
    ref_g = [t.grad.clone() for t in leaves]
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
    grads = [t.grad for t in leaves]
    for i in range(3):
        noise = torch.randn(4096, device="cuda")
        (noise * noise).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), f"{case}: replay {i} output {k}"
        for k, (a, b) in enumerate(zip(grads, ref_g)):
            assert torch.equal(a, b), f"{case}: replay {i} gradient {k}"


@pytest.mark.parametrize("n", [64, 128])
def test_wkv7_operator_graph_replay(hip_lib, n):
    # N = 128: the sequential kernels over row-split workgroups, whose
    # partial column sums take stream-ordered memory from the library's pool
    # (a memory node in the captured graph)
    import rwkv7m_amd
    from rwkv7m_amd.kernels.wkv_ffi import unregister_wkv_ffi_backend
    print(f"case: wkv7 graph replay T70 B2 H2 N{n} bf16", flush=True)
    inp = make_inputs(70, 2, 2, n, seed=41, state_std=0.1)
    leaves = [inp[n].cuda().requires_grad_(True) for n in NAMES]
    s0 = inp["s0"].cuda().requires_grad_(True)
    dy = inp["dy"].cuda()
    unregister_wkv_ffi_backend()
    rwkv7m_amd.register_hip_backend()
    try:
        def step():
            y, s_t = rwkv7m_amd.wkv7(*leaves, s0, "ffi")
            ((y.float() * dy.float()).sum() + s_t.sum()).backward()
            return [y, s_t]

        _replay_check(step, leaves + [s0], f"wkv7 N{n}")
    finally:
        unregister_wkv_ffi_backend()


def test_time_mix_wkv_graph_replay(hip_lib):
    from rwkv7m_amd.timemix import time_mix_wkv
    print("case: time_mix_wkv graph replay B2 T40 H2 N64 bf16", flush=True)
    B, T, H, N = 2, 40, 2, 64
    C = H * N
    g = torch.Generator(device="cuda").manual_seed(3)

    def act(scale=1.0):
        return (torch.randn(B, T, C, device="cuda", generator=g) * scale).to(
            torch.bfloat16).requires_grad_(True)

    r, w_raw, k, v, gate = act(), act(0.5), act(), act(), act()
    a = torch.sigmoid(torch.randn(B, T, C, device="cuda", generator=g)).to(
        torch.bfloat16).requires_grad_(True)
    par = [torch.full((C,), x, device="cuda").requires_grad_(True)
           for x in (0.7, 1.02, -0.04, 0.8, 0.0)]
    dout = torch.randn(B, T, C, device="cuda", generator=g)

    def step():
        out, s_t = time_mix_wkv(r, w_raw, k, v, a, gate, *par, n_heads=H)
        ((out.float() * dout).sum() + s_t.sum()).backward()
        return [out, s_t]

    _replay_check(step, [r, w_raw, k, v, a, gate] + par, "time_mix_wkv")
