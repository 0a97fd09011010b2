"""Host-side logic on the CPU: the operator API, backend policy, FFI registry,
the C-ABI library's exports and argument checks, and the oracle against the
committed golden fixtures.

Mirrors the reference's tests/test_wkv_api.py and the registry/policy tests
of tests/test_wkv_pallas.py:113-198 with torch in place of JAX.  Nothing here
launches GPU work.
"""

import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

import oracle
from rwkv7m_amd.kernels.wkv_backend import resolve_wkv_backend
from rwkv7m_amd.kernels.wkv_ffi import (WKVFFIBackend,
                                        register_wkv_ffi_backend,
                                        unregister_wkv_ffi_backend)
from rwkv7m_amd.wkv import wkv7, wkv7_batch_major, wkv7_reference

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
NAMES = ("r", "w", "k", "v", "neg_kk", "kka")
GRAD_NAMES = ("dr", "dw", "dk", "dv", "dneg_kk", "dkka", "ds0")


def _inputs(dtype=torch.float32, time=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    vecs = tuple((torch.randn(time, 1, 2, 4, generator=g) * 0.1).to(dtype)
                 for _ in range(6))
    state = torch.randn(1, 2, 4, 4, generator=g) * 0.1
    return (*vecs, state)


def _np(t):
    return t.detach().float().numpy().astype(np.float64)


# ---------------------------------------------------------------------------
# Operator API (reference tests/test_wkv_api.py)
# ---------------------------------------------------------------------------

def test_wkv7_reference_matches_oracle_and_dtype_contract():
    inputs = _inputs(torch.bfloat16)
    y, s_t = wkv7_reference(*inputs)
    assert y.dtype == torch.bfloat16 and s_t.dtype == torch.float32
    ey, es = oracle.forward(*(_np(x) for x in inputs))
    np.testing.assert_allclose(_np(s_t), es, rtol=1e-5, atol=1e-6)
    # y is rounded to bf16 once, after the fp32 scan
    np.testing.assert_array_equal(
        _np(y), _np(torch.from_numpy(ey).to(torch.bfloat16)))


def test_wkv7_custom_vjp_matches_oracle_gradients():
    inputs = [x.clone().requires_grad_(True) for x in _inputs()]
    y, s_t = wkv7(*inputs)
    loss = (y.square().sum() + 0.01 * s_t.square().sum())
    grads = torch.autograd.grad(loss, inputs)
    dy = 2 * _np(y)
    ds_t = 0.02 * _np(s_t)
    expected = oracle.backward(*(_np(x) for x in inputs), dy, ds_t)
    for name, g, e in zip(GRAD_NAMES, grads, expected):
        np.testing.assert_allclose(_np(g), e, rtol=1e-5, atol=1e-6,
                                   err_msg=name)


def test_wkv7_rejects_invalid_shapes_and_dtypes():
    *vecs, s0 = _inputs()
    with pytest.raises(TypeError, match="initial_state must be float32"):
        wkv7_reference(*vecs, s0.to(torch.bfloat16))
    with pytest.raises(ValueError, match="k must have shape"):
        wkv7_reference(vecs[0], vecs[1], vecs[2][:, :, :, :-1], *vecs[3:],
                       s0)
    with pytest.raises(TypeError, match="bfloat16 or float32"):
        wkv7_reference(*(x.to(torch.float16) for x in vecs), s0)


def test_wkv7_documents_reverse_mode_only_contract():
    inputs = [x.clone().requires_grad_(True) for x in _inputs()]
    tangents = tuple(torch.ones_like(x) for x in inputs)
    with pytest.raises(TypeError, match="forward-mode autodiff"):
        torch.func.jvp(lambda *xs: wkv7(*xs), tuple(inputs), tangents)


# ---------------------------------------------------------------------------
# Backend policy and FFI registry (reference tests/test_wkv_pallas.py:113-198)
# ---------------------------------------------------------------------------

def test_auto_backend_is_pallas_first_and_never_selects_ffi(monkeypatch):
    monkeypatch.delenv("RWKV7M_WKV_BACKEND", raising=False)
    assert resolve_wkv_backend(platform="cpu") == "reference"
    assert resolve_wkv_backend(platform="tpu") == "pallas_tpu"
    assert resolve_wkv_backend(platform="gpu",
                               device_kind="NVIDIA L40S") == \
        "pallas_gpu_triton"
    assert resolve_wkv_backend(platform="gpu",
                               device_kind="NVIDIA H100 80GB HBM3") == \
        "pallas_gpu_mosaic"


def test_backend_environment_override_is_validated(monkeypatch):
    monkeypatch.setenv("RWKV7M_WKV_BACKEND", "ffi")
    assert resolve_wkv_backend(platform="cpu") == "ffi"
    monkeypatch.setenv("RWKV7M_WKV_BACKEND", "not-a-backend")
    with pytest.raises(ValueError, match="unknown WKV backend"):
        resolve_wkv_backend(platform="cpu")


def test_ffi_requires_explicit_registration():
    unregister_wkv_ffi_backend()
    with pytest.raises(RuntimeError, match="no FFI backend is registered"):
        wkv7(*_inputs(), "ffi")


def test_registered_ffi_satisfies_forward_and_backward_contract():
    calls = []

    def forward(*values):
        calls.append("forward")
        return wkv7_reference(*values)

    def forward_with_aux(*values):
        calls.append("forward_with_aux")
        return wkv7_reference(*values), (torch.tensor(7),)

    def backward(*values):
        calls.append("backward")
        primal, cot, aux = values[:7], values[7:9], values[9:]
        assert len(aux) == 1 and int(aux[0]) == 7
        with torch.enable_grad():
            xs = [x.detach().requires_grad_(True) for x in primal]
            outs = wkv7_reference(*xs)
            return torch.autograd.grad(outs, xs, grad_outputs=cot)

    backend = WKVFFIBackend(forward=forward,
                            forward_with_aux=forward_with_aux,
                            backward=backward)
    unregister_wkv_ffi_backend()
    register_wkv_ffi_backend(backend)
    try:
        with pytest.raises(RuntimeError, match="already registered"):
            register_wkv_ffi_backend(backend)
        register_wkv_ffi_backend(backend, replace=True)
        inputs = _inputs()
        with torch.no_grad():
            actual = wkv7(*inputs, "ffi")
        expected = wkv7_reference(*inputs)
        assert all(torch.equal(a, e) for a, e in zip(actual, expected))
        assert calls == ["forward"]

        xs = [x.clone().requires_grad_(True) for x in inputs]
        got = torch.autograd.grad(wkv7(*xs, "ffi")[0].sum(), xs)
        ys = [x.clone().requires_grad_(True) for x in inputs]
        want = torch.autograd.grad(wkv7_reference(*ys)[0].sum(), ys)
        assert all(torch.allclose(a, b) for a, b in zip(got, want))
        assert calls[1:] == ["forward_with_aux", "backward"]
    finally:
        unregister_wkv_ffi_backend()


def _batch_inputs(dtype=torch.float32, seed=3):
    """Batch-major [B=2, T=5, H=2, N=4] vectors and a [2, 2, 4, 4] state."""
    g = torch.Generator().manual_seed(seed)
    vecs = tuple((torch.randn(2, 5, 2, 4, generator=g) * 0.3).to(dtype)
                 for _ in range(6))
    return (*vecs, torch.randn(2, 2, 4, 4, generator=g) * 0.1)


def test_wkv7_batch_major_equals_transposes_around_wkv7():
    # the reference's time-mix layer: swap axes 0 and 1 of the six vectors,
    # call wkv7, swap y back (nnx_model.py:695-698, :709-711)
    inputs = _batch_inputs()
    y, s_t = wkv7_batch_major(*inputs, "reference")
    ty, ts = wkv7_reference(*(x.transpose(0, 1) for x in inputs[:6]),
                            inputs[6])
    assert y.shape == inputs[0].shape
    assert torch.equal(y, ty.transpose(0, 1)) and torch.equal(s_t, ts)
    # against the oracle on the time-major copies
    ey, es = oracle.forward(*(_np(x.transpose(0, 1)) for x in inputs[:6]),
                            _np(inputs[6]))
    np.testing.assert_allclose(_np(y.transpose(0, 1)), ey, rtol=1e-5,
                               atol=1e-6)
    np.testing.assert_allclose(_np(s_t), es, rtol=1e-5, atol=1e-6)

    xs = [x.clone().requires_grad_(True) for x in inputs]
    y, s_t = wkv7_batch_major(*xs, "reference")
    got = torch.autograd.grad((y * y).sum() + s_t.sum(), xs)
    zs = [x.clone().requires_grad_(True) for x in inputs]
    ty, ts = wkv7_reference(*(z.transpose(0, 1) for z in zs[:6]), zs[6])
    want = torch.autograd.grad((ty * ty).sum() + ts.sum(), zs)
    for a, b in zip(got, want):
        assert a.shape == b.shape and torch.allclose(a, b, atol=1e-6)


def test_wkv7_batch_major_other_ffi_backends_get_time_major_vectors():
    # an FFI backend other than the HIP kernels sees the reference's
    # time-major contract: the transposes run around it
    shapes = []

    def forward(*values):
        shapes.append(tuple(values[0].shape))
        return wkv7_reference(*values)

    backend = WKVFFIBackend(forward=forward,
                            forward_with_aux=lambda *a: (forward(*a), ()),
                            backward=None)
    unregister_wkv_ffi_backend()
    register_wkv_ffi_backend(backend)
    try:
        inputs = _batch_inputs()
        with torch.no_grad():
            y, s_t = wkv7_batch_major(*inputs, "ffi")
        assert shapes == [(5, 2, 2, 4)]
        ey, es = wkv7_batch_major(*inputs, "reference")
        assert torch.equal(y, ey) and torch.equal(s_t, es)
    finally:
        unregister_wkv_ffi_backend()


def test_wkv7_batch_major_validates_batch_major_shapes():
    inputs = list(_batch_inputs())
    with pytest.raises(ValueError, match="batch, time, heads"):
        wkv7_batch_major(inputs[0][0], *inputs[1:], "reference")
    bad = inputs.copy()
    bad[3] = bad[3][:, :4]
    with pytest.raises(ValueError, match=r"\(2, 5, 2, 4\)"):
        wkv7_batch_major(*bad, "reference")
    bad = inputs.copy()
    bad[2] = bad[2].to(torch.bfloat16)
    with pytest.raises(TypeError, match="all WKV vectors"):
        wkv7_batch_major(*bad, "reference")


# ---------------------------------------------------------------------------
# C ABI: the library loads on a host without a GPU and exports the header
# ---------------------------------------------------------------------------

def _declared_functions():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(rwkv7m_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    from rwkv7m_amd import _build
    from rwkv7m_amd.kernels import wkv_hip
    if not os.path.exists(wkv_hip.LIB_PATH):
        _build.build()
    return wkv_hip.load_library()


def test_library_exports_every_declared_symbol(lib):
    from rwkv7m_amd.kernels import wkv_hip
    declared = _declared_functions()
    assert declared, "no declarations found in include/*.h"
    assert declared == set(wkv_hip.EXPORTED_SYMBOLS)
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert lib.rwkv7m_abi_version() == 1


def test_library_host_queries(lib):
    assert lib.rwkv7m_wkv7_checkpoint_count(0, 16) == 1
    assert lib.rwkv7m_wkv7_checkpoint_count(5, 2) == 4
    assert lib.rwkv7m_wkv7_checkpoint_count(4096, 32) == 129
    assert lib.rwkv7m_wkv7_checkpoint_count(-1, 16) == -1
    assert lib.rwkv7m_wkv7_checkpoint_count(5, 0) == -1
    assert lib.rwkv7m_wkv7_default_checkpoint_interval(1, 64) == 16
    assert lib.rwkv7m_wkv7_default_checkpoint_interval(0, 64) == 16
    # bf16 checkpoints exactly for the MFMA-served intervals
    for ci in (0, 16, 32, 64):
        assert lib.rwkv7m_wkv7_checkpoint_dtype(1, 64, ci) == 1
    for dtype, n, ci in ((1, 64, 8), (1, 64, 128), (1, 32, 16),
                         (0, 64, 32), (0, 16, 0)):
        assert lib.rwkv7m_wkv7_checkpoint_dtype(dtype, n, ci) == 0


def test_library_rejects_bad_requests_before_any_device_call(lib):
    null = [None] * 10
    assert lib.rwkv7m_wkv7_forward(5, 1, 1, 1, 4, *null) == 1
    assert b"bfloat16 or float32" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_forward(0, 1, 1, 1, 48, *null) == 2
    assert lib.rwkv7m_wkv7_forward(0, 2, 1, 1, 4, *null) == 1
    assert b"is NULL" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_forward_with_aux(
        0, 2, 1, 1, 4, *null, -1, None) == 1
    assert b"checkpoint_interval" in lib.rwkv7m_last_error()
    # the batch-major entry points check the same things and name themselves
    assert lib.rwkv7m_wkv7_forward_bthn(0, 2, 1, 1, 4, *null) == 1
    assert b"rwkv7m_wkv7_forward_bthn" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_forward_with_aux_bthn(
        1, 2, 1, 1, 4, *null, 0, None) == 1
    assert b"checkpoints is NULL" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_backward_bthn(
        0, 2, 1, 1, 4, *null, -1, *([None] * 8)) == 1
    assert b"rwkv7m_wkv7_backward_bthn" in lib.rwkv7m_last_error()


def test_summed_backward_checks_its_arguments_before_any_device_call(lib):
    # rwkv7m_timemix_wkv_backward: the backward's own checks (named after
    # the entry point), then an added cotangent that is an output buffer is
    # refused; the fake addresses below are never dereferenced
    fake = [ctypes.c_void_p(0x1000 * (i + 1)) for i in range(10)]
    outs = [ctypes.c_void_p(0x100000 * (i + 1)) for i in range(7)]
    fn = lib.rwkv7m_timemix_wkv_backward
    assert fn(1, 2, 1, 1, 64, *fake, -1, None, None, None, *outs, None) == 1
    assert b"rwkv7m_timemix_wkv_backward: checkpoint_interval" in \
        lib.rwkv7m_last_error()
    assert fn(1, 2, 1, 1, 64, *fake, 16, None, None, None, *outs[:6], None,
              None) == 1
    assert b"ds0 is NULL" in lib.rwkv7m_last_error()
    for i, o in ((0, 0), (1, 2), (2, 3), (0, 3), (2, 5)):
        adds = [None, None, None]
        adds[i] = outs[o]
        assert fn(1, 2, 1, 1, 64, *fake, 16, *adds, *outs, None) == 1
        assert b"may not overlap an output buffer" in lib.rwkv7m_last_error()
    # a partly overlapping view is refused as well: the check compares byte
    # ranges (the vectors are 2 * 64 bf16 = 256 bytes here)
    for shift in (8, -8, 248, -248):
        adds = [None, ctypes.c_void_p(outs[4].value + shift), None]
        assert fn(1, 2, 1, 1, 64, *fake, 16, *adds, *outs, None) == 1
        assert b"may not overlap an output buffer" in lib.rwkv7m_last_error()
    assert lib.rwkv7m_wkv7_last_path() == b""


def test_backward_refuses_ds0_sharing_bytes_with_ds_t(lib):
    # The exact pass of a marked head reads dS_T after dS0 holds the mark,
    # so dS0 may not share a byte with dS_T: the same buffer and partly
    # overlapping views are refused before any device call (the fake
    # addresses are never dereferenced; states are 64 * 64 * 4 bytes)
    # r, w, k, v, neg_kk, kka, initial_state, dy; then the checkpoints
    fake = [ctypes.c_void_p(0x1000 * (i + 1)) for i in range(9)]
    outs = [ctypes.c_void_p(0x100000 * (i + 1)) for i in range(6)]
    ds_t = 0x4000000
    for entry in (lib.rwkv7m_wkv7_backward, lib.rwkv7m_wkv7_backward_bthn):
        for shift in (0, 4, 16380, -16380):
            ds0 = ctypes.c_void_p(ds_t + shift)
            rc = entry(1, 2, 1, 1, 64, *fake[:8], ctypes.c_void_p(ds_t),
                       fake[8], 16, *outs, ds0, None)
            assert rc == 1
            assert b"ds0 may not overlap ds_t" in lib.rwkv7m_last_error()
        assert lib.rwkv7m_wkv7_last_path() == b""


def test_noalloc_consumer_backward_rejects_sizes_beyond_its_scratch(lib):
    # 2^22 channels need more partial rows than the built-in scratch holds:
    # rejected by the size check, before any pointer is used or any device
    # is touched (the fake addresses below are never dereferenced)
    fake = [ctypes.c_void_p(0x1000 * (i + 1)) for i in range(17)]
    rc = lib.rwkv7m_timemix_wkv_output_backward_noalloc(
        1, 4, 1 << 15, 128, *fake[:8], 64e-5, *fake[8:], None)
    assert rc == 1
    assert b"built-in scratch" in lib.rwkv7m_last_error()


def test_last_path_is_empty_after_a_rejected_call(lib):
    # the path query names only kernels a successful call launched
    null = [None] * 10
    assert lib.rwkv7m_wkv7_forward(0, 2, 1, 1, 4, *null) == 1
    assert lib.rwkv7m_wkv7_last_path() == b""
    assert lib.rwkv7m_wkv7_backward(
        0, 2, 1, 1, 4, *null, 0, *([None] * 8)) == 1
    assert lib.rwkv7m_wkv7_last_path() == b""
    # the wait-budget hook takes any value without touching a device
    lib.rwkv7m_debug_set_wait_limit(1)
    lib.rwkv7m_debug_set_wait_limit(0)


def test_timemix_abi_checks_requests_before_any_device_call(lib):
    # workspace: one partial row of C floats per row group for 3 parameters
    assert lib.rwkv7m_timemix_workspace_floats(0, 32, 64) == 3 * 2048
    assert lib.rwkv7m_timemix_workspace_floats(1, 32, 64) == 3 * 2048
    assert lib.rwkv7m_timemix_workspace_floats(32768, 32, 64) == \
        3 * 1024 * 2048
    assert lib.rwkv7m_timemix_workspace_floats(-1, 32, 64) == -1
    assert lib.rwkv7m_timemix_workspace_floats(8, 2, 4) == -1
    fake = 1 << 20  # aligned, never dereferenced: every call below fails
    odd = fake + 8  # not 16-byte aligned
    p9 = [fake] * 9
    fn = lib.rwkv7m_timemix_wkv_inputs
    assert fn(2, 4, 2, 64, *p9, None) == 1
    assert b"bfloat16 or float32" in lib.rwkv7m_last_error()
    assert fn(1, 4, 2, 4, *p9, None) == 2
    assert b"(8, 16, 32, 64, 128)" in lib.rwkv7m_last_error()
    assert fn(1, -1, 2, 64, *p9, None) == 1
    assert fn(1, 4, 2, 64, *p9[:3], None, *p9[4:], None) == 1
    assert b"k_k is NULL" in lib.rwkv7m_last_error()
    assert fn(1, 4, 2, 64, *p9[:5], odd, *p9[6:], None) == 1
    assert b"w is not 16-byte aligned" in lib.rwkv7m_last_error()
    # nothing to do: no rows, or no heads
    assert fn(1, 0, 2, 64, *([None] * 9), None) == 0
    assert fn(1, 4, 0, 64, *([None] * 9), None) == 0
    bwd = lib.rwkv7m_timemix_wkv_inputs_backward
    ws = lib.rwkv7m_timemix_workspace_floats(4, 2, 64)
    args16 = [fake] * 16
    assert bwd(1, 4, 2, 64, *args16, ws - 1, None) == 1
    assert b"workspace holds" in lib.rwkv7m_last_error()
    assert bwd(1, 4, 2, 64, *args16[:15], None, ws, None) == 1
    assert b"workspace is NULL" in lib.rwkv7m_last_error()
    out = lib.rwkv7m_timemix_wkv_output
    assert out(1, 4, 2, 64, *([fake] * 8), -1.0, fake, None) == 1
    assert b"eps" in lib.rwkv7m_last_error()
    assert out(1, 4, 2, 64, *([fake] * 8), float("nan"), fake, None) == 1
    assert out(1, 4, 2, 64, *([fake] * 8), 64e-5, None, None) == 1
    assert b"out is NULL" in lib.rwkv7m_last_error()
    obwd = lib.rwkv7m_timemix_wkv_output_backward
    assert obwd(1, 4, 2, 64, *([fake] * 8), 64e-5, *([fake] * 5), None,
                *([fake] * 3), None, 0, None) == 1
    assert b"workspace holds 0" in lib.rwkv7m_last_error()
    assert obwd(1, 4, 2, 64, *([fake] * 8), 64e-5, *([fake] * 5), None,
                *([fake] * 3), fake, 10 ** 9, None) == 1
    assert b"dg is NULL" in lib.rwkv7m_last_error()


# ---------------------------------------------------------------------------
# Oracle against the committed golden fixtures
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN,
                                                               "*.npz"))),
                         ids=os.path.basename)
def test_oracle_reproduces_golden_fixture(path):
    data = np.load(path)
    bf16 = bool(data["is_bf16"])

    def vec(name):
        x = data[name]
        return (oracle.bf16_from_bits(x) if bf16 else x).astype(np.float64)

    vecs = [vec(n) for n in NAMES]
    s0 = data["s0"].astype(np.float64)
    y, s_t = oracle.forward(*vecs, s0)
    np.testing.assert_allclose(y, data["y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s_t, data["s_t"], rtol=1e-5, atol=1e-6)
    if "dr" in data:
        grads = oracle.backward(*vecs, s0, vec("dy"),
                                data["ds_t"].astype(np.float64))
        for name, g in zip(GRAD_NAMES, grads):
            np.testing.assert_allclose(g, data[name], rtol=1e-5, atol=1e-6,
                                       err_msg=name)


def test_screening_abi_checks_requests_before_any_device_call(lib):
    # workspace: three [chunks][B][M][ds] fp32 arrays, 32 steps per chunk
    assert lib.rwkv7m_screen_slot_scan_workspace_floats(8, 512, 16, 128) == \
        3 * 16 * 8 * 16 * 128
    assert lib.rwkv7m_screen_slot_scan_workspace_floats(2, 0, 4, 64) == \
        3 * 2 * 4 * 64
    assert lib.rwkv7m_screen_slot_scan_workspace_floats(-1, 8, 4, 64) == -1
    fake = 1 << 20
    scan = lib.rwkv7m_screen_slot_scan
    assert scan(3, 2, 8, 4, 64, *([fake] * 8), 10 ** 6, None) == 1
    assert b"bfloat16 or float32" in lib.rwkv7m_last_error()
    assert scan(1, 2, 8, 4, 64, *([fake] * 8), 10, None) == 1
    assert b"workspace holds 10" in lib.rwkv7m_last_error()
    assert scan(1, 2, 8, 4, 64, fake, None, *([fake] * 6), 10 ** 6,
                None) == 1
    assert b"slot_term is NULL" in lib.rwkv7m_last_error()
    assert scan(1, 0, 8, 4, 64, *([None] * 8), 0, None) == 0  # no batch
    read = lib.rwkv7m_screen_read
    args = [fake, fake, fake, 1e-6, None, 0, 1, 0, 0.0, 8.0, 1.0, 1e-6]
    assert read(1, 2, 8, 65, 64, 64, *args, *([fake] * 4), None) == 2
    assert b"M <= 64" in lib.rwkv7m_last_error()
    assert read(1, 2, 8, 16, 64, 600, *args, *([fake] * 4), None) == 2
    bad_cap = args[:10] + [0.0] + args[11:]
    assert read(1, 2, 8, 16, 64, 64, *bad_cap, *([fake] * 4), None) == 1
    assert b"cap" in lib.rwkv7m_last_error()
    no_tau = args[:2] + [None] + args[3:]
    assert read(1, 2, 8, 16, 64, 64, *no_tau, *([fake] * 4), None) == 1
    assert b"tau is NULL" in lib.rwkv7m_last_error()
    bwd = lib.rwkv7m_screen_read_backward
    assert bwd(1, 2, 8, 16, 64, 64, *args, fake, None, None,
               *([fake] * 3), None) == 1
    assert b"dq is NULL" in lib.rwkv7m_last_error()


def test_screening_write_abi_checks_requests_before_any_device_call(lib):
    fake = 1 << 20
    write = lib.rwkv7m_screen_write
    ins = [fake] * 7  # base, slot_term, slot_embed, kw, q_w, tau_w, mu
    outs = [fake] * 9  # slots0, ages0, slots_seq, .., slots_T, ages_T
    for ds, dk, msg in ((2048, 64, b"ds <= 1024"), (128, 200, b"dk <= 128"),
                        (128, 0, b"1 <= dk")):
        assert write(1, 2, 8, 4, ds, dk, *ins, 0.05, 1e-6, *outs,
                     None) == 2, (ds, dk)
        assert msg in lib.rwkv7m_last_error()
    assert write(1, 2, 8, 4, 128, 64, *ins, -0.1, 1e-6, *outs, None) == 1
    assert b"floor and eps" in lib.rwkv7m_last_error()
    assert write(3, 2, 8, 4, 128, 64, *ins, 0.05, 1e-6, *outs, None) == 1
    assert b"bfloat16 or float32" in lib.rwkv7m_last_error()
    no_kw = ins[:3] + [None] + ins[4:]
    assert write(1, 2, 8, 4, 128, 64, *no_kw, 0.05, 1e-6, *outs,
                 None) == 1
    assert b"kw is NULL" in lib.rwkv7m_last_error()
    no_q = ins[:4] + [None] + ins[5:]
    assert write(1, 2, 8, 4, 128, 64, *no_q, 0.05, 1e-6, *outs, None) == 1
    assert b"q_w is NULL" in lib.rwkv7m_last_error()
    # no batch rows or no slots: nothing to do, no pointer read
    assert write(1, 0, 8, 4, 128, 64, *([None] * 7), 0.05, 1e-6,
                 *([None] * 9), None) == 0
    bwd = lib.rwkv7m_screen_write_backward
    bouts = [fake] * 8  # d_pre, d_slots0, .., d_tau_w
    cots = [fake, fake, None, None, None]  # slots32, d_slots_seq, optional
    assert bwd(1, 2, 8, 4, 128, 0, *ins, 0.05, 1e-6, *cots, None, *bouts,
               None) == 2
    assert b"1 <= dk" in lib.rwkv7m_last_error()
    no_dpre = [None] + bouts[1:]
    assert bwd(1, 2, 8, 4, 128, 64, *ins, 0.05, 1e-6, *cots, None,
               *no_dpre, None) == 1
    assert b"d_pre is NULL" in lib.rwkv7m_last_error()


def test_screening_config_checks_follow_the_reference():
    """ScreeningConfig.__post_init__ rejects what the reference's does, with
    its messages (src/rwkv7m/model/screening.py:124-140), and the module's
    compute dtype defaults to float32 as NNXStateLevelScreening's does."""
    from rwkv7m_amd.screening import ScreeningConfig, StateLevelScreening
    base = dict(d_model=16, d_slot=8, d_k=4, d_v=4, n_slots=2)
    for bad in (1.0, -0.1, 1.5):
        with pytest.raises(ValueError, match=r"usage_ema_decay must be in "
                                             r"\[0, 1\)"):
            ScreeningConfig(**base, usage_ema_decay=bad)
    ScreeningConfig(**base, usage_ema_decay=0.0)
    for field in ("short_half_life_tokens", "mid_half_life_tokens",
                  "long_half_life_tokens"):
        with pytest.raises(ValueError, match="memory half-life values must "
                                             "be positive when provided"):
            ScreeningConfig(**base, **{field: 0.0})
    with pytest.raises(ValueError, match="bank_ids must have length n_slots"):
        ScreeningConfig(**base, bank_ids=(0,))
    with pytest.raises(ValueError, match="bank_ids values must be only"):
        ScreeningConfig(**base, bank_ids=(0, 3))
    with pytest.raises(ValueError, match="write_rel_floor must be"):
        ScreeningConfig(**base, write_rel_floor=-1.0)
    mod = StateLevelScreening(ScreeningConfig(**base))
    assert mod.compute_dtype == torch.float32


def test_hip_wrappers_check_shapes_dtypes_and_devices_first(lib):
    # the ctypes wrappers hand the kernels bare pointers: a shorter vector,
    # a state of the wrong shape or dtype, or a host tensor is refused
    # before any call (no GPU needed)
    from rwkv7m_amd.kernels import wkv_hip
    T, B, H, N = 3, 2, 2, 64
    vec = [torch.zeros(T, B, H, N, dtype=torch.bfloat16) for _ in range(6)]
    s0 = torch.zeros(B, H, N, N)
    short = list(vec)
    short[1] = torch.zeros(T - 1, B, H, N, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="w has shape"):
        wkv_hip.forward(*short, s0)
    mixed = list(vec)
    mixed[4] = vec[4].float()
    with pytest.raises(ValueError, match="neg_kk has shape"):
        wkv_hip.forward_with_aux(*mixed, s0)
    with pytest.raises(ValueError, match="initial_state has shape"):
        wkv_hip.forward(*vec, torch.zeros(B, H, N, N - 1))
    with pytest.raises(TypeError, match="initial_state must be float32"):
        wkv_hip.forward(*vec, s0.double())
    with pytest.raises(RuntimeError, match="needs GPU tensors"):
        wkv_hip.forward(*vec, s0)
    with pytest.raises(ValueError, match="state must be a float32"):
        wkv_hip.decode_inplace(*(v[:1] for v in vec), torch.zeros(B, H, N, 2))


def test_screening_wrappers_check_shapes_and_devices_first(lib):
    # the screening entry points take bare pointers too: mismatched shapes
    # and host tensors are refused before any call (no GPU needed)
    from rwkv7m_amd.kernels import screening_hip as sh
    B, T, M, ds, dk = 2, 5, 3, 8, 4
    base = torch.zeros(B, T, ds)
    with pytest.raises(ValueError, match="slots0 has shape"):
        sh.slot_scan(base, torch.zeros(M, ds), torch.zeros(M),
                     torch.zeros(B, M, ds + 1))
    with pytest.raises(ValueError, match="mu has shape"):
        sh.slot_scan(base, torch.zeros(M, ds), torch.zeros(M + 1),
                     torch.zeros(B, M, ds))
    with pytest.raises(RuntimeError, match="needs GPU tensors"):
        sh.slot_scan(base, torch.zeros(M, ds), torch.zeros(M),
                     torch.zeros(B, M, ds))
    with pytest.raises(ValueError, match="k_proj_w has shape"):
        sh.write(base, torch.zeros(M, ds), torch.zeros(M, ds),
                 torch.zeros(ds + 1, dk), torch.zeros(B, T, dk),
                 torch.zeros(()), torch.zeros(M), 1e-3, 1e-6,
                 torch.zeros(B, M, ds), torch.zeros(B, M))
    with pytest.raises(ValueError, match="tau_w must hold one value"):
        sh.write(base, torch.zeros(M, ds), torch.zeros(M, ds),
                 torch.zeros(ds, dk), torch.zeros(B, T, dk),
                 torch.zeros(2), torch.zeros(M), 1e-3, 1e-6,
                 torch.zeros(B, M, ds), torch.zeros(B, M))
