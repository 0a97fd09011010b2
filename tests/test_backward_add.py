"""GPU: the WKV-7 backward with added cotangents
(``rwkv7m_timemix_wkv_backward``, ``wkv_hip.backward(..., add=...)``).

The time mix's r, k' and v also feed its consumer, so their cotangents are
sums of two terms (nnx_model.py:695-727 under jax autodiff).  The summed
backward adds the consumer's terms to dr, dk and dv in fp32 before its own
rounding.  Checked against the plain batch-major backward on the same
inputs, on every kernel path (wave backward at each interval, a head handed
to the exact sequential pass, the sequential kernels for fp32 and for an
interval the wave kernels do not serve):

* dw, dneg_kk, dkka and dS0, and any gradient whose added cotangent is
  None, are bit-identical to the plain backward;
* dr, dk, dv equal plain + added within the two roundings that separate
  them: |got - (plain + add)| <= u (|plain + add| + |plain|) elementwise,
  u the unit roundoff of the vector dtype.  A cotangent added at the wrong
  token, channel or head misses this by about its own size.
"""

import pytest
import torch

from rwkv7m_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")
# (case, T, B, H, N, dtype, interval, strong decay, expected backward path)
CASES = [
    ("wave L16 T100", 100, 2, 3, 64, torch.bfloat16, 16, False,
     "wave_backward"),
    ("wave L32 T70", 70, 2, 2, 64, torch.bfloat16, 32, False,
     "wave_backward"),
    ("wave L64 T130", 130, 1, 3, 64, torch.bfloat16, 64, False,
     "wave_backward"),
    ("exact pass L16 T80", 80, 1, 3, 64, torch.bfloat16, 16, True,
     "wave_backward"),
    ("exact pass L32 T75", 75, 2, 3, 64, torch.bfloat16, 32, True,
     "wave_backward"),
    ("exact pass L64 T140", 140, 1, 3, 64, torch.bfloat16, 64, True,
     "wave_backward"),
    ("sequential fp32 N16 T23", 23, 2, 2, 16, torch.float32, 16, False,
     "seq_backward"),
    ("sequential L128 T150", 150, 1, 2, 64, torch.bfloat16, 128, False,
     "seq_backward"),
]


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip


def _bm(t):
    """[T, B, H, N] -> batch-major [B, T, H, N] on the GPU."""
    return t.transpose(0, 1).contiguous().cuda()


def _check_sum(name, got, plain, add, u, case):
    exp = plain.float() + add.float()
    bound = u * (exp.abs() + plain.float().abs()) + 1e-30
    err = (got.float() - exp).abs()
    worst = float((err / bound).max())
    assert worst <= 1.0, f"{case} {name}: error {worst:.3f} x the bound"


@pytest.mark.parametrize("case,T,B,H,N,dtype,ci,strong,path", CASES,
                         ids=[c[0] for c in CASES])
def test_summed_backward_equals_plain_plus_added(hip, case, T, B, H, N,
                                                 dtype, ci, strong, path):
    print("case:", case, flush=True)
    inp = make_inputs(T, B, H, N, dtype=dtype, seed=T + N + ci,
                      state_std=0.1, dstate_std=0.1)
    if strong:
        # exp(w) ~ 7 per token in head 1: the wave backward hands that head
        # to the exact sequential pass
        w = inp["w"].float()
        w[:, :, 1] += 3.0
        inp["w"] = w.to(dtype)
    vecs = [_bm(inp[n]) for n in NAMES]
    s0, ds_t = inp["s0"].cuda(), inp["ds_t"].cuda()
    dy = _bm(inp["dy"])
    (_, _), aux = hip.forward_with_aux(*vecs, s0, checkpoint_interval=ci,
                                       layout="bthn")
    plain = hip.backward(*vecs, s0, dy, ds_t, *aux, layout="bthn")
    assert hip.last_path() == path, (case, hip.last_path())
    g = torch.Generator().manual_seed(T)
    adds = []
    for i in (0, 2, 3):  # dr, dk, dv
        scale = float(plain[i].float().abs().max())
        adds.append((torch.randn(vecs[0].shape, generator=g) * scale).to(
            dtype).cuda())
    summed = hip.backward(*vecs, s0, dy, ds_t, *aux, layout="bthn",
                          add=tuple(adds))
    assert hip.last_path() == path, (case, hip.last_path())
    # dk's cotangent left out: dk is the plain one, bit for bit
    partial = hip.backward(*vecs, s0, dy, ds_t, *aux, layout="bthn",
                           add=(adds[0], None, adds[2]))
    torch.cuda.synchronize()
    hip.device_status()
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -24
    for i, name in ((1, "dw"), (4, "dneg_kk"), (5, "dkka"), (6, "ds0")):
        assert torch.equal(summed[i], plain[i]), (case, name)
        assert torch.equal(partial[i], plain[i]), (case, name)
    for j, (i, name) in enumerate(((0, "dr"), (2, "dk"), (3, "dv"))):
        _check_sum(name, summed[i], plain[i], adds[j], u, case)
    assert torch.equal(partial[2], plain[2]), (case, "dk without add")
    assert torch.equal(partial[0], summed[0]), (case, "dr")
    assert torch.equal(partial[3], summed[3]), (case, "dv")


def test_summed_backward_needs_batch_major_vectors(hip):
    inp = make_inputs(20, 1, 1, 64, seed=3)
    vecs = [inp[n].cuda() for n in NAMES]
    s0 = inp["s0"].cuda()
    (_, _), aux = hip.forward_with_aux(*vecs, s0)
    with pytest.raises(ValueError, match="batch-major"):
        hip.backward(*vecs, s0, inp["dy"].cuda(), None, *aux,
                     add=(vecs[0], None, None))


def test_summed_backward_at_the_headline_shape(hip):
    # config 2's shape in the model's batch-major layout, the wave backward
    # at the default interval, every head
    from rwkv7m_amd.synthetic import config_inputs
    case = "summed backward B8 T4096 H32 N64 bf16 batch-major"
    print("case:", case, flush=True)
    inp = config_inputs(2, device="cuda", generator="torch")
    vecs = [inp[n].transpose(0, 1).contiguous() for n in NAMES]
    dy = inp["dy"].transpose(0, 1).contiguous()
    s0, ds_t = inp["s0"], inp["ds_t"]
    del inp
    (_, _), aux = hip.forward_with_aux(*vecs, s0, layout="bthn")
    plain = hip.backward(*vecs, s0, dy, ds_t, *aux, layout="bthn")
    g = torch.Generator(device="cuda").manual_seed(7)
    adds = [torch.randn(vecs[0].shape, generator=g, device="cuda").mul_(
        float(plain[i].float().abs().max())).to(torch.bfloat16)
        for i in (0, 2, 3)]
    summed = hip.backward(*vecs, s0, dy, ds_t, *aux, layout="bthn",
                          add=tuple(adds))
    assert hip.last_path() == "wave_backward"
    torch.cuda.synchronize()
    hip.device_status()
    for i, name in ((1, "dw"), (4, "dneg_kk"), (5, "dkka"), (6, "ds0")):
        assert torch.equal(summed[i], plain[i]), (case, name)
    for j, (i, name) in enumerate(((0, "dr"), (2, "dk"), (3, "dv"))):
        _check_sum(name, summed[i], plain[i], adds[j], 2.0 ** -8, case)
