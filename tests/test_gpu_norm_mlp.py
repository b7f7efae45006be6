"""SwiGLU and RMSNorm kernels on the GPU against the float64 oracle, through the C ABI
(the prefixlm.swiglu / prefixlm.rms_norm custom ops).

Bar: every output is within 1.02 * 2^-8 of the oracle relative to the size of the
terms it sums: one bf16 rounding of an fp32 result (half an ulp is at most 2^-8
relative, at the bottom of a binade) plus 2% for fp32 arithmetic error; the autograd
path gives the same bits as the direct ops.
Shapes: config 5 (16384 x 5632 SwiGLU, 16384 x 2048 RMSNorm), tiny and ragged rows,
every register-chunk variant of the norm (1 to 16 chunks per lane), strided views.
"""
import numpy as np
import pytest
import torch

from oracle import norm_mlp_oracle as orc
from prefixlm import rms_norm, swiglu
from prefixlm.norm_mlp import rms_norm_bwd, rms_norm_fwd, swiglu_bwd, swiglu_fwd

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
EPS = 1e-6
REL = 1.02 * 2.0 ** -8


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _check(tag, got, ref, size):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    bound = REL * size + 1e-6
    worst = float((err / bound).max()) if err.size else 0.0
    print(f"[parity] {tag}: max_abs={err.max() if err.size else 0:.3e} worst/bound={worst:.3f}", flush=True)
    assert worst <= 1.0, tag


@pytest.mark.parametrize("rows,F", [(16384, 5632), (1, 8), (37, 40), (3, 1000)])
def test_swiglu_fwd_bwd(rows, F):
    print(f"[case] swiglu rows={rows} F={F}", flush=True)
    gu = _bf16((rows, 2 * F), 10 + rows, 2.0)
    dy = _bf16((rows, F), 20 + rows)
    g64, d64 = gu.double().numpy(), dy.double().numpy()
    y = swiglu_fwd(gu.to(DEV))
    dgu = swiglu_bwd(gu.to(DEV), dy.to(DEV))
    torch.cuda.synchronize()
    ref_y = orc.swiglu_fwd(g64)
    _check(f"swiglu fwd {rows}x{F}", y, ref_y, np.abs(ref_y))
    ref_d = orc.swiglu_bwd(g64, d64)
    _check(f"swiglu bwd {rows}x{F}", dgu, ref_d, np.abs(ref_d))


def test_swiglu_strided_rows_and_autograd():
    rows, F = 64, 256
    big = _bf16((rows, 2 * F + 64), 3, 2.0).to(DEV)
    gu = big[:, 16:16 + 2 * F]          # row stride 2F + 64, 32-byte offset
    assert gu.stride(0) == 2 * F + 64
    dy = _bf16((rows, F), 4).to(DEV)
    y = swiglu_fwd(gu)
    _check("swiglu fwd strided", y, orc.swiglu_fwd(gu.double().cpu().numpy()),
           np.abs(orc.swiglu_fwd(gu.double().cpu().numpy())))
    t = gu.detach().clone().requires_grad_()
    out = swiglu(t)
    out.backward(dy)
    assert torch.equal(out, swiglu_fwd(gu))
    assert torch.equal(t.grad, swiglu_bwd(gu, dy))


@pytest.mark.parametrize("rows,cols", [(16384, 2048), (5, 8), (33, 520), (9, 1024), (7, 4096), (7, 8192),
                                       (2, 4104)])
def test_rms_norm_fwd_bwd(rows, cols):
    print(f"[case] rms_norm rows={rows} cols={cols}", flush=True)
    x = _bf16((rows, cols), 30 + cols, 3.0)
    dy = _bf16((rows, cols), 40 + cols)
    x64, d64 = x.double().numpy(), dy.double().numpy()
    y, rstd = rms_norm_fwd(x.to(DEV), EPS)
    dx = rms_norm_bwd(x.to(DEV), rstd, dy.to(DEV))
    torch.cuda.synchronize()
    ref_y, ref_r = orc.rms_norm_fwd(x64, EPS)
    _check(f"rms_norm fwd {rows}x{cols}", y, ref_y, np.abs(ref_y))
    np.testing.assert_allclose(rstd.cpu().numpy(), ref_r, rtol=1e-5)
    ref_dx = orc.rms_norm_bwd(x64, ref_r, d64)
    r = ref_r[:, None]
    size = np.abs(r * d64) + np.abs(x64 * r ** 3 * np.mean(d64 * x64, axis=-1, keepdims=True))
    _check(f"rms_norm bwd {rows}x{cols}", dx, ref_dx, size)


def test_rms_norm_zero_rows_and_autograd():
    x = _bf16((16, 256), 5).to(DEV)
    x[3] = 0                            # a zero row normalises to zero, r = eps^-1/2
    y, rstd = rms_norm_fwd(x, EPS)
    assert torch.count_nonzero(y[3]) == 0
    assert abs(rstd[3].item() - EPS ** -0.5) <= 1e-3 * EPS ** -0.5
    dy = _bf16((16, 256), 6).to(DEV)
    t = x.detach().clone().requires_grad_()
    out = rms_norm(t, EPS)
    out.backward(dy)
    assert torch.equal(out, y)
    assert torch.equal(t.grad, rms_norm_bwd(x, rstd, dy))
    e = rms_norm_fwd(torch.empty((0, 64), dtype=torch.bfloat16, device=DEV), EPS)
    assert e[0].shape == (0, 64) and e[1].shape == (0,)
