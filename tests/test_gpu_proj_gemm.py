"""The projection GEMM with the RMSNorm and the SwiGLU fused in (prefixlm_proj_gemm,
csrc/gemm.h) against float64: the oracle's RMSNorm and SwiGLU (oracle/norm_mlp_oracle.py)
around a float64 matrix product.

Bar: |y - ref| <= 1.02 * 2^-8 * |ref| (one bf16 rounding of the fp32 result) plus
2^-18 times the size of the summed terms (fp32 accumulation over K and the fp32 row
scale): size = r * (|x| |W|^T) for a plain projection, and for the SwiGLU output
|d silu(g)/dg * u| * size_g + |silu(g)| * size_u. The unfused bf16 path (norm, GEMM,
SwiGLU as separate roundings) is reported beside it.
Shapes: config 5 (16384 x 2048 against the 11264 x 2048 gate_up weight and the
8192 x 2048 gqkv weight), ragged row counts, a strided x."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import norm_mlp_oracle as orc
from prefixlm.norm_mlp import proj_gemm

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
EPS = 1e-6


def _data(M, K, N, seed, x_stride=None):
    g = torch.Generator(device="cpu").manual_seed(seed)
    xs = x_stride or K
    xbuf = torch.randn(M, xs, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    return xbuf[:, :K], w


def _reference(x, w, swiglu, norm):
    xd = x.double()
    if norm:
        h, r = orc.rms_norm_fwd(xd.cpu().numpy(), EPS)
        hd = torch.from_numpy(h).to(DEV)
        rd = torch.from_numpy(r).to(DEV)[:, None]
    else:
        hd, rd = xd, torch.ones((x.shape[0], 1), dtype=torch.float64, device=DEV)
    y = hd @ w.double().t()
    size = rd * (xd.abs() @ w.double().abs().t())
    if not swiglu:
        return y, size
    Fh = w.shape[0] // 2
    ref = torch.from_numpy(orc.swiglu_fwd(y.cpu().numpy())).to(DEV)
    gg, sg, su = y[:, :Fh], size[:, :Fh], size[:, Fh:]
    s = torch.sigmoid(gg)
    dsilu = s * (1 + gg * (1 - s))
    return ref, (dsilu * y[:, Fh:]).abs() * sg + (gg * s).abs() * su


@pytest.mark.parametrize("swiglu,N", [(True, 11264), (False, 8192)])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("M,x_stride", [(16384, None), (1000, None), (1, None), (300, 2056)])
def test_proj_gemm_against_float64(swiglu, N, norm, M, x_stride):
    K = 2048
    x, w = _data(M, K, N, seed=M + N + (7 if norm else 0), x_stride=x_stride)
    y = proj_gemm(x, w, swiglu, norm, EPS)
    torch.cuda.synchronize()
    ref, size = _reference(x, w, swiglu, norm)
    err = (y.double() - ref).abs()
    bound = 1.02 * 2.0 ** -8 * ref.abs() + 2.0 ** -18 * size + 1e-12
    worst = (err / bound).max().item()
    h = F.rms_norm(x, (K,), eps=EPS) if norm else x
    yu = F.linear(h, w)
    if swiglu:
        g_, u_ = yu.chunk(2, dim=-1)
        yu = F.silu(g_) * u_
    err_u = (yu.double() - ref).abs()
    print(f"[parity] proj_gemm swiglu={swiglu} norm={norm} M={M}: max_abs={err.max().item():.3e} "
          f"worst/bound={worst:.3f} (unfused bf16 path max_abs={err_u.max().item():.3e}) "
          f"max|ref|={ref.abs().max().item():.3f}", flush=True)
    assert worst <= 1.0
    assert err.max().item() <= err_u.max().item() + 1e-6


def test_stack_with_fused_projections_without_grad():
    """The config-5 stack (all bf16, one layer per module) with the norms fused into the
    gqkv and gate_up projections and the SwiGLU into the latter (no-grad forward, the
    reference's mode for all but the last bp_steps module calls): within the floor the
    bf16 stack with PyTorch's ops already shows against the float32 stack."""
    from oracle.prefixlm_oracle import attention_fwd
    from prefixlm import flash_attn_varlen_prefixlm
    from prefixlm.hrm_stack import HRMStack, HRMStackConfig, packed_position_ids
    from prefixlm.synth import metadata_tensors, segments_for_config
    prefix, causal = segments_for_config(5)
    T = 16384
    st, ss = metadata_tensors(prefix, causal, T, DEV)
    seq = {**st, **ss}
    pos = packed_position_ids(prefix, causal, T, DEV)
    segs, cs = [], 0
    for p, c in zip(prefix, causal):
        segs.append((cs, int(p), int(p + c)))
        cs += int(p + c)
    base = HRMStack(HRMStackConfig(layers_per_module=1)).init_weights(1005)
    x = torch.randn(T, 2048, generator=torch.Generator(device="cpu").manual_seed(1005)).to(torch.bfloat16).to(DEV)

    def model(dtype, **flags):
        m = HRMStack(HRMStackConfig(layers_per_module=1, **flags)).to(DEV)
        with torch.no_grad():
            for (_, p), (_, p0) in zip(m.named_parameters(), base.named_parameters()):
                p.copy_(p0.to(torch.bfloat16).float())
            m.zL_init.copy_(base.zL_init)
        return m.to(dtype)

    def ref_attn(q, k, v, is_causal, **_):
        return attention_fwd(q, k, v, segs, is_causal)[0].to(q.dtype)
    with torch.no_grad():
        out_ref = model(torch.float32)(x.float(), pos, ref_attn, seq)
        out_plain = model(torch.bfloat16)(x, pos, flash_attn_varlen_prefixlm, seq)
        out_fused = model(torch.bfloat16, fused_elementwise=True, fused_gemm=True)(
            x, pos, flash_attn_varlen_prefixlm, seq)
    torch.cuda.synchronize()
    e_plain = (out_plain.float() - out_ref).abs().max().item()
    e_fused = (out_fused.float() - out_ref).abs().max().item()
    print(f"[parity] cfg5 stack no-grad: fused projections {e_fused:.3e}, PyTorch ops {e_plain:.3e} "
          f"(vs fp32 stack, max|ref|={out_ref.abs().max().item():.3f})", flush=True)
    assert torch.isfinite(out_fused).all()
    assert e_fused <= max(3e-2, 1.5 * e_plain)
