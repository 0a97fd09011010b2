"""The MFMA kernels split over several workgroups per head.

Forward: with few heads the library splits each head's chunks over two
workgroups: each writes y and the checkpoints of its own run of chunks and
first carries the state through the chunks before them
(rwkv7m_debug_set_forward_segments overrides the count).  Every count must
give y, S_T and checkpoints bit-identical to one workgroup per head.

Backward:

With few heads (B * H well below the CU count) the library splits each
head's chunks over up to four workgroups: each writes the gradients of its
own run of chunks and first carries the cotangent through the chunks after
them (rwkv7m_debug_set_backward_segments overrides the count).  The split
changes no arithmetic, so every count must give results bit-identical to one
workgroup per head (an interval of 32 tokens is never split: one workgroup
per head takes the decay gradient's boundary sums at the checkpoint chunks,
which a segment's first chunk cannot follow): for every checkpoint interval,
a ragged final chunk,
nonzero initial state and state cotangent, the summing (time-mix) instance,
heads that the exact sequential pass takes over, and the automatic count at
config 1's shape (B8 T512 H12: 96 heads on 256 CUs).  The oracle parity of
the split path itself is covered by every small-shape test of
test_chunked_parity.py, which now runs split by default.
"""

import pytest
import torch

from rwkv7m_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("r", "w", "k", "v", "neg_kk", "kka")


@pytest.fixture(scope="module")
def hip(hip_lib):
    from rwkv7m_amd.kernels import wkv_hip
    yield wkv_hip
    wkv_hip.set_backward_segments(0)
    wkv_hip.set_forward_segments(0)


def _forward(hip, dev, ci, segments):
    hip.set_forward_segments(segments)
    vecs = [dev[n] for n in NAMES]
    (y, s_t), (ckpt, _) = hip.forward_with_aux(*vecs, dev["s0"],
                                               checkpoint_interval=ci)
    assert hip.last_path() == "wave_forward"
    torch.cuda.synchronize()
    return [y.clone(), s_t.clone(), ckpt.clone()]


def _compare_forward(hip, inp, ci, counts, case):
    print("case:", case, flush=True)
    dev = {k: v.cuda() for k, v in inp.items()}
    ref = _forward(hip, dev, ci, 1)
    for k in counts:
        got = _forward(hip, dev, ci, k)
        for name, a, b in zip(("y", "S_T", "checkpoints"), got, ref):
            assert torch.equal(a, b), (
                f"{case}: {k} workgroups per head, {name} differs from one "
                f"workgroup per head")
    hip.set_forward_segments(0)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_forward_split_is_bit_identical(hip, ci):
    for T, B, H in ((1000, 1, 2), (130, 2, 1), (40, 1, 3)):
        inp = make_inputs(T, B, H, 64, seed=T + ci, state_std=0.1)
        _compare_forward(hip, inp, ci, (0, 2),
                         f"forward split T{T} B{B} H{H} L{ci}")


def test_forward_split_with_exact_chunks(hip):
    # decays strong in tokens 256..383 of head 1: those chunks take the
    # chains' exact pass, in the first segment's own chunks and in the
    # second's carried ones
    inp = make_inputs(768, 1, 2, 64, seed=13, state_std=0.1)
    w = inp["w"].float()
    w[256:384, :, 1] += 3.0
    inp["w"] = w.to(torch.bfloat16)
    _compare_forward(hip, inp, 16, (0, 2), "forward split exact chunks")


def test_forward_split_config1_shape(hip):
    inp = make_inputs(512, 8, 12, 64, seed=1, generator="torch")
    _compare_forward(hip, inp, 16, (0,), "forward split config 1")


def _backward(hip, dev, aux, segments, layout, add=None):
    hip.set_backward_segments(segments)
    vecs = [dev[n] for n in NAMES]
    g = hip.backward(*vecs, dev["s0"], dev["dy"], dev["ds_t"], *aux,
                     layout=layout, add=add)
    assert hip.last_path() == "wave_backward"
    torch.cuda.synchronize()
    return [t.clone() for t in g]


def _compare(hip, inp, ci, counts, case, add=False):
    print("case:", case, flush=True)
    dev = {k: v.cuda() for k, v in inp.items()}
    layout = "tbhn"
    extra = None
    if add:
        # the summing instance takes batch-major vectors
        layout = "bthn"
        for n in NAMES + ("dy",):
            dev[n] = dev[n].transpose(0, 1).contiguous()
        gen = torch.Generator(device="cuda").manual_seed(3)
        extra = [torch.randn(dev["r"].shape, generator=gen,
                             device="cuda").to(torch.bfloat16)
                 for _ in range(3)]
    vecs = [dev[n] for n in NAMES]
    (_, _), aux = hip.forward_with_aux(*vecs, dev["s0"],
                                       checkpoint_interval=ci, layout=layout)
    ref = _backward(hip, dev, aux, 1, layout, extra)
    for k in counts:
        got = _backward(hip, dev, aux, k, layout, extra)
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), (
                f"{case}: {k} workgroups per head, output {i} differs from "
                f"one workgroup per head")
    hip.set_backward_segments(0)


@pytest.mark.parametrize("ci", [16, 32, 64])
def test_split_is_bit_identical(hip, ci):
    # 63 chunks (ragged last one) for L = 16; the planner keeps interval
    # boundaries and falls back to fewer segments where it must
    T = 1000 if ci == 16 else 1024
    inp = make_inputs(T, 1, 2, 64, seed=70 + ci, state_std=0.1,
                      dstate_std=0.1)
    _compare(hip, inp, ci, (0, 2, 3, 4), f"split T{T} B1 H2 L{ci}")


def test_split_is_bit_identical_short_sequences(hip):
    for T in (40, 96, 130):
        inp = make_inputs(T, 2, 1, 64, seed=T, state_std=0.1,
                          dstate_std=0.1)
        _compare(hip, inp, 16, (0, 2, 4), f"split T{T} B2 H1 L16")


def test_split_summing_instance(hip):
    # the time mix's instance adds the consumer's cotangents of r, k, v
    inp = make_inputs(512, 1, 3, 64, seed=9, state_std=0.1, dstate_std=0.1)
    _compare(hip, inp, 16, (2, 4), "split summing T512 B1 H3 L16", add=True)


def test_split_with_exact_pass_heads(hip):
    # decays strong in tokens 256..383 of head 1 only: that head goes to
    # the exact sequential pass whichever workgroup meets the chunk first
    inp = make_inputs(768, 1, 2, 64, seed=12, state_std=0.1, dstate_std=0.1)
    w = inp["w"].float()
    w[256:384, :, 1] += 3.0
    inp["w"] = w.to(torch.bfloat16)
    _compare(hip, inp, 16, (0, 2, 3, 4), "split exact-pass head T768 L16")


def test_split_config1_shape(hip):
    # B8 T512 H12: 96 heads; the default count splits them
    inp = make_inputs(512, 8, 12, 64, seed=1, generator="torch")
    _compare(hip, inp, 16, (0,), "split config 1 B8 T512 H12 L16")
