"""The consumer backward's no-allocation entry point
(rwkv7m_timemix_wkv_output_backward_noalloc) against the workspace entry
point it varies (rwkv7m_timemix_wkv_output_backward).

Both run the same kernels; the no-allocation one takes its partial-row
scratch from the library's built-in device array instead of a caller
workspace.  Two calls in a row, the second with a smaller input, must each
give results bit-identical to the workspace entry point's: the second call
reads only scratch entries it wrote itself.  A third call with fp32
activations covers the other dtype.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tm(hip_lib):
    from rwkv7m_amd.kernels import timemix_hip
    return timemix_hip


def _inputs(rows, H, N, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    C = H * N

    def act(scale=1.0, shift=0.0):
        return (torch.randn(rows, C, generator=g, device="cuda") * scale +
                shift).to(dtype)

    acts = [act(0.7, 0.3), act(), act(), act(), act(), act()]  # y r k v g dout
    params = [-0.04 + 0.3 * torch.randn(C, generator=g, device="cuda"),
              1.0 + 0.1 * torch.randn(C, generator=g, device="cuda"),
              0.1 * torch.randn(C, generator=g, device="cuda")]
    return acts, params


@pytest.mark.parametrize("rows,H,N,dtype", [
    (8 * 4096, 32, 64, torch.bfloat16),   # config 2's rows: the full scratch
    (300, 12, 64, torch.bfloat16),        # smaller: reads only what it wrote
    (77, 5, 32, torch.float32),
], ids=["c2-bf16", "small-bf16", "small-f32"])
def test_noalloc_matches_workspace_entry_point(tm, rows, H, N, dtype):
    print(f"case: consumer backward no-alloc rows={rows} H={H} N={N} "
          f"{dtype}", flush=True)
    (y, r, k, v, g, dout), (r_k, sc, bi) = _inputs(rows, H, N, dtype,
                                                  seed=rows + N)
    ref = tm.output_backward(y, r, k, v, g, r_k, sc, bi, dout, N)
    out = [torch.full_like(y, float("nan")) for _ in range(4)] + [
        torch.full_like(g, float("nan"))] + [
        torch.full((H * N,), float("nan"), device="cuda") for _ in range(3)]
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    got = tm.output_backward_noalloc(y, r, k, v, g, r_k, sc, bi, dout, N,
                                     out=out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    names = ("dy", "dr", "dk", "dv", "dg", "dr_k", "dln_scale", "dln_bias")
    for name, a, b in zip(names, got, ref):
        assert a.data_ptr() in [o.data_ptr() for o in out]
        assert torch.equal(a, b), f"{name} differs from the workspace call"
