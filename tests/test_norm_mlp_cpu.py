"""SwiGLU / RMSNorm without a GPU: the float64 oracle pinned against PyTorch's own CPU
routines, autograd and finite differences (with planted mistakes that the checks
must catch), the custom ops' fake shapes and torch.compile tracing, and the C ABI's
argument validation (no compute calls)."""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import norm_mlp_oracle as orc
from prefixlm import _build, _capi
from prefixlm.norm_mlp import rms_norm_fwd, swiglu_fwd

EPS = 1e-6


def _rng(seed):
    return np.random.default_rng(seed)


def _swiglu_torch(gu):
    g, u = gu.chunk(2, dim=-1)
    return F.silu(g) * u


def test_swiglu_fwd_matches_torch():
    gu = _rng(1).standard_normal((7, 48)) * 3.0
    ref = _swiglu_torch(torch.from_numpy(gu)).numpy()
    np.testing.assert_allclose(orc.swiglu_fwd(gu), ref, rtol=1e-13, atol=1e-14)


def test_swiglu_extreme_gates_do_not_overflow():
    gu = np.array([[-800.0, 800.0, 0.0, 2.0, 3.0, -1.0]])
    y = orc.swiglu_fwd(gu)
    assert np.all(np.isfinite(y))
    np.testing.assert_allclose(y, [[-0.0, 800.0 * 3.0, 0.0]], atol=1e-12)


def test_swiglu_bwd_matches_autograd():
    r = _rng(2)
    gu = r.standard_normal((5, 32)) * 2.0
    dy = r.standard_normal((5, 16))
    t = torch.from_numpy(gu).requires_grad_()
    (ref,) = torch.autograd.grad(_swiglu_torch(t), t, torch.from_numpy(dy))
    np.testing.assert_allclose(orc.swiglu_bwd(gu, dy), ref.numpy(), rtol=1e-12, atol=1e-13)


def _fd(fn, x, dy, h=1e-6):
    """Central finite differences of sum(fn(x) * dy) with respect to x."""
    g = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = (np.sum(fn(xp) * dy) - np.sum(fn(xm) * dy)) / (2 * h)
    return g


def test_swiglu_bwd_finite_differences_and_planted_mistake():
    r = _rng(3)
    gu = r.standard_normal((3, 16)) * 2.0
    dy = r.standard_normal((3, 8))
    fd = _fd(orc.swiglu_fwd, gu, dy)
    np.testing.assert_allclose(orc.swiglu_bwd(gu, dy), fd, rtol=1e-6, atol=1e-7)
    # a dropped term in the gate's derivative (silu' taken as sigmoid) is caught
    F8 = 8
    g, u = gu[:, :F8], gu[:, F8:]
    s = 1 / (1 + np.exp(-g))
    wrong = np.concatenate([dy * u * s, dy * g * s], axis=-1)
    assert not np.allclose(wrong, fd, rtol=1e-3, atol=1e-4)


def test_swiglu_closed_form_at_zero_gate():
    u = _rng(4).standard_normal((2, 8))
    gu = np.concatenate([np.zeros_like(u), u], axis=-1)
    dy = np.ones_like(u)
    np.testing.assert_array_equal(orc.swiglu_fwd(gu), np.zeros_like(u))
    d = orc.swiglu_bwd(gu, dy)
    np.testing.assert_allclose(d[:, :8], 0.5 * u, rtol=1e-15)   # silu'(0) = 1/2
    np.testing.assert_array_equal(d[:, 8:], np.zeros_like(u))   # silu(0) = 0


def test_rms_norm_fwd_matches_torch():
    x = _rng(5).standard_normal((6, 40)) * 4.0
    y, rstd = orc.rms_norm_fwd(x, EPS)
    ref = F.rms_norm(torch.from_numpy(x), (40,), eps=EPS).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(rstd, 1 / np.sqrt((x * x).mean(-1) + EPS), rtol=1e-14)


def test_rms_norm_constant_row():
    for c in (-3.0, 1e-4, 250.0):
        y, _ = orc.rms_norm_fwd(np.full((1, 16), c), EPS)
        np.testing.assert_allclose(y, np.full((1, 16), c / np.sqrt(c * c + EPS)), rtol=1e-14)


def test_rms_norm_bwd_matches_autograd_and_finite_differences():
    r = _rng(6)
    x = r.standard_normal((4, 24)) * 2.0
    dy = r.standard_normal((4, 24))
    _, rstd = orc.rms_norm_fwd(x, EPS)
    got = orc.rms_norm_bwd(x, rstd, dy)
    t = torch.from_numpy(x).requires_grad_()
    (ref,) = torch.autograd.grad(F.rms_norm(t, (24,), eps=EPS), t, torch.from_numpy(dy))
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-11, atol=1e-12)
    fd = _fd(lambda z: orc.rms_norm_fwd(z, EPS)[0], x, dy)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-7)
    # the r^3 cross term is what makes dx orthogonal to x's direction; without it the
    # finite differences disagree
    assert not np.allclose(rstd[:, None] * dy, fd, rtol=1e-3, atol=1e-4)


def test_fake_shapes_and_compile_trace():
    gu = torch.empty((5, 3, 64), dtype=torch.bfloat16, device="meta")
    assert swiglu_fwd(gu).shape == (5, 3, 32)
    x = torch.empty((5, 3, 64), dtype=torch.bfloat16, device="meta")
    y, rstd = rms_norm_fwd(x, EPS)
    assert y.shape == x.shape and rstd.shape == (15,) and rstd.dtype == torch.float32

    from prefixlm import rms_norm, swiglu

    def f(gu, x):
        return swiglu(gu).sum() + rms_norm(x, EPS).sum()

    out = torch.compile(f, backend="eager", fullgraph=True)(gu, x)
    assert out.shape == ()


@pytest.fixture(scope="module")
def lib():
    import os
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    return _capi.load()


def test_capi_validation(lib):
    fake = 1 << 20   # never dereferenced: validation fails first
    a = _capi.SwigluArgs(fake, fake, fake, fake, 64, 32, 32, 64, 4, 12)
    assert lib.prefixlm_swiglu_fwd(ctypes.byref(a), None) == 1
    assert "multiple of 8" in _capi.last_error()
    a = _capi.SwigluArgs(fake, fake, fake, fake, 16, 8, 8, 16, 4, 16)   # gu stride 16 < 2 * cols
    assert lib.prefixlm_swiglu_bwd(ctypes.byref(a), None) == 1
    assert "row stride" in _capi.last_error()
    a = _capi.SwigluArgs(fake + 2, None, fake, None, 64, 32, 0, 0, 4, 32)
    assert lib.prefixlm_swiglu_fwd(ctypes.byref(a), None) == 1
    assert "aligned" in _capi.last_error()
    a = _capi.RmsnormArgs(fake, fake, fake, fake, fake, 8200, 8200, 8200, 8200, 4, 8200, EPS)
    assert lib.prefixlm_rmsnorm_fwd(ctypes.byref(a), None) == 1
    assert "multiple of 8" in _capi.last_error()
    a = _capi.RmsnormArgs(fake, fake, fake, fake, None, 64, 64, 64, 64, 4, 64, EPS)
    assert lib.prefixlm_rmsnorm_bwd(ctypes.byref(a), None) == 1
    assert "rstd" in _capi.last_error()
    a = _capi.RmsnormArgs(fake, None, fake, None, fake, 64, 64, 0, 0, 0, 64, EPS)
    assert lib.prefixlm_rmsnorm_fwd(ctypes.byref(a), None) == 0   # no rows: nothing to launch
