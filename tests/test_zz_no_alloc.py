"""The consumer backward's no-allocation entry point
(rwkv7m_timemix_wkv_output_backward_noalloc) against the workspace entry
point it varies (rwkv7m_timemix_wkv_output_backward).

Both run the same kernels; the no-allocation one takes its partial-row
scratch from the library's built-in device array instead of a caller
workspace.  Two calls in a row, the second with a smaller input, must each
give results bit-identical to the workspace entry point's: the second call
reads only scratch entries it wrote itself.  A third call with fp32
activations covers the other dtype.  Around each call the device's free
memory (hipMemGetInfo) must not move, which a hipMalloc inside the library
would show and torch's own allocator statistics would not.

The entry point is also offered to code under graph capture, and its first
call on a device looks the scratch up.  A fresh process therefore makes its
first call under torch.cuda.graph, replays the graph several times with eager
calls in between that overwrite the scratch, and checks every replay bit for
bit against the workspace entry point.
"""

import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def tm(hip_lib):
    from rwkv7m_amd.kernels import timemix_hip
    # one call first: it looks the scratch up (and may load the code object
    # that holds it), which the free-memory checks below must not count
    (y, r, k, v, g, dout), (r_k, sc, bi) = _inputs(4, 2, 64, torch.bfloat16, 1)
    timemix_hip.output_backward_noalloc(y, r, k, v, g, r_k, sc, bi, dout, 64)
    torch.cuda.synchronize()
    return timemix_hip


def _free_bytes():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]


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
    free_before = _free_bytes()
    got = tm.output_backward_noalloc(y, r, k, v, g, r_k, sc, bi, dout, N,
                                     out=out)
    free_after = _free_bytes()
    assert torch.cuda.memory_allocated() == before
    assert free_after == free_before, (
        f"device free memory moved by {free_before - free_after} bytes")
    names = ("dy", "dr", "dk", "dv", "dg", "dr_k", "dln_scale", "dln_bias")
    for name, a, b in zip(names, got, ref):
        assert a.data_ptr() in [o.data_ptr() for o in out]
        assert torch.equal(a, b), f"{name} differs from the workspace call"


# Run in a child process so that the captured call is the process's first
# call of the entry point (the one that looks the scratch up).
_CAPTURE = r"""
import sys
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
from rwkv7m_amd.kernels import wkv_hip, timemix_hip as tm
from test_zz_no_alloc import _inputs

wkv_hip.load_library()
rows, H, N = 300, 12, 64
(y, r, k, v, g, dout), (r_k, sc, bi) = _inputs(rows, H, N, torch.bfloat16, 7)
ref = tm.output_backward(y, r, k, v, g, r_k, sc, bi, dout, N)
out = [torch.empty_like(y) for _ in range(4)] + [torch.empty_like(g)] + [
    torch.empty(H * N, device="cuda") for _ in range(3)]
# a second, larger input for the eager calls between replays: they
# overwrite the scratch rows the graph reads
(y2, r2, k2, v2, g2, dout2), (rk2, sc2, bi2) = _inputs(
    4 * rows, H, N, torch.bfloat16, 8)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    tm.output_backward_noalloc(y, r, k, v, g, r_k, sc, bi, dout, N, out=out)
torch.cuda.synchronize()
names = ("dy", "dr", "dk", "dv", "dg", "dr_k", "dln_scale", "dln_bias")
for rep in range(3):
    for o in out:
        o.fill_(float("nan"))
    tm.output_backward_noalloc(y2, r2, k2, v2, g2, rk2, sc2, bi2, dout2, N)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(names, out, ref):
        assert torch.equal(a, b), f"replay {rep}: {name} differs"
    print(f"replay {rep}: bit-identical", flush=True)
print("capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(hip_lib):
    print("case: consumer backward no-alloc, first call captured in a "
          "graph, 3 replays (child process)", flush=True)
    res = subprocess.run([sys.executable, "-c", _CAPTURE, ROOT],
                         capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stderr[-2000:]
    assert "capture ok" in res.stdout
