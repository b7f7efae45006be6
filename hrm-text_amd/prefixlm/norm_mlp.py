"""SwiGLU activation and weightless RMSNorm of the HRM block as HIP kernels.

The reference's block computes ``F.silu(gate) * up`` on the two halves of the gate/up
projection (models/layers.py:166-168) and ``F.rms_norm(x, (N,), eps)`` before the
attention and the MLP and after the last layer (models/transformer.py:87, :90-92,
:116). As PyTorch ops that is a silu, a multiply, and in the backward two more
elementwise kernels plus a concatenation that assembles the projection's gradient
from its two halves; RMSNorm's backward reads its inputs in several passes.

``swiglu`` and ``rms_norm`` run each direction as one kernel: one pass over the
inputs and outputs, fp32 arithmetic and one bf16 rounding per output (autograd
rounds the SwiGLU product and its gradients twice). The SwiGLU backward writes the
gradient of the whole [rows, 2F] projection output.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch
from torch import Tensor

from . import _capi
from .op import _ptr, _stream

__all__ = ["swiglu", "rms_norm", "swiglu_fwd", "swiglu_bwd", "rms_norm_fwd", "rms_norm_bwd", "proj_gemm",
           "rms_norm_linear", "rms_norm_swiglu"]


def _rows(x: Tensor, name: str) -> Tensor:
    """x as a bf16 [rows, cols] GPU view with unit column stride and 16-byte aligned rows."""
    if x.dtype != torch.bfloat16 or x.device.type != "cuda" or x.dim() < 1:
        raise ValueError(f"{name} must be a bf16 GPU tensor (got {x.dtype} {tuple(x.shape)} on {x.device})")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


@torch.library.custom_op("prefixlm::swiglu_fwd", mutates_args=())
def swiglu_fwd(gu: Tensor) -> Tensor:
    """silu(gate) * up for gu [..., 2F] = [gate | up] -> [..., F]."""
    if gu.shape[-1] % 16:
        raise ValueError(f"the last dimension of gu (2F = {gu.shape[-1]}) must be a multiple of 16")
    lib = _capi.load()
    g2 = _rows(gu, "gu")
    F = g2.shape[1] // 2
    y = torch.empty((g2.shape[0], F), dtype=gu.dtype, device=gu.device)
    a = _capi.SwigluArgs(_ptr(g2), None, _ptr(y), None, g2.stride(0), y.stride(0), 0, 0, g2.shape[0], F)
    with torch.cuda.device(gu.device):
        _capi.check(lib.prefixlm_swiglu_fwd(ctypes.byref(a), _stream(gu.device)), "prefixlm_swiglu_fwd")
    return y.view(*gu.shape[:-1], F)


@swiglu_fwd.register_fake
def _swiglu_fwd_fake(gu):
    return gu.new_empty((*gu.shape[:-1], gu.shape[-1] // 2))


@torch.library.custom_op("prefixlm::swiglu_bwd", mutates_args=())
def swiglu_bwd(gu: Tensor, dy: Tensor) -> Tensor:
    """Gradient of swiglu_fwd with respect to gu, [..., 2F]."""
    if gu.shape[-1] % 16 or tuple(dy.shape) != (*gu.shape[:-1], gu.shape[-1] // 2):
        raise ValueError(f"gu {tuple(gu.shape)} and dy {tuple(dy.shape)} do not match")
    lib = _capi.load()
    g2, d2 = _rows(gu, "gu"), _rows(dy, "dy")
    F = g2.shape[1] // 2
    dgu = torch.empty(g2.shape, dtype=gu.dtype, device=gu.device)
    a = _capi.SwigluArgs(_ptr(g2), _ptr(d2), None, _ptr(dgu), g2.stride(0), 0, d2.stride(0), dgu.stride(0),
                         g2.shape[0], F)
    with torch.cuda.device(gu.device):
        _capi.check(lib.prefixlm_swiglu_bwd(ctypes.byref(a), _stream(gu.device)), "prefixlm_swiglu_bwd")
    return dgu.view(gu.shape)


@swiglu_bwd.register_fake
def _swiglu_bwd_fake(gu, dy):
    return gu.new_empty(gu.shape)


class SwiGLUFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gu):
        ctx.save_for_backward(gu)
        return swiglu_fwd(gu)

    @staticmethod
    def backward(ctx, dy):
        (gu,) = ctx.saved_tensors
        return swiglu_bwd(gu, dy)


def swiglu(gu: Tensor) -> Tensor:
    """``F.silu(gate) * up`` with ``gate, up = gu.chunk(2, dim=-1)`` (models/layers.py:167-168)."""
    return SwiGLUFunction.apply(gu)


@torch.library.custom_op("prefixlm::rms_norm_fwd", mutates_args=())
def rms_norm_fwd(x: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    """(y, rstd): y = x * rstd over the last dimension, rstd fp32 [rows]."""
    lib = _capi.load()
    x2 = _rows(x, "x")
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    rstd = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    a = _capi.RmsnormArgs(_ptr(x2), None, _ptr(y), None, _ptr(rstd), x2.stride(0), y.stride(0), 0, 0,
                          x2.shape[0], x2.shape[1], float(eps))
    with torch.cuda.device(x.device):
        _capi.check(lib.prefixlm_rmsnorm_fwd(ctypes.byref(a), _stream(x.device)), "prefixlm_rmsnorm_fwd")
    return y.view(x.shape), rstd


@rms_norm_fwd.register_fake
def _rms_norm_fwd_fake(x, eps):
    rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
    return x.new_empty(x.shape), x.new_empty((rows,), dtype=torch.float32)


@torch.library.custom_op("prefixlm::rms_norm_bwd", mutates_args=())
def rms_norm_bwd(x: Tensor, rstd: Tensor, dy: Tensor) -> Tensor:
    """dx = rstd * dy - x * rstd^3 * mean(dy * x) over the last dimension."""
    if tuple(dy.shape) != tuple(x.shape):
        raise ValueError(f"x {tuple(x.shape)} and dy {tuple(dy.shape)} do not match")
    lib = _capi.load()
    x2, d2 = _rows(x, "x"), _rows(dy, "dy")
    if rstd.dtype != torch.float32 or rstd.numel() != x2.shape[0]:
        raise ValueError(f"rstd must be float32 [{x2.shape[0]}] (got {rstd.dtype} {tuple(rstd.shape)})")
    rstd = rstd.contiguous()
    dx = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    a = _capi.RmsnormArgs(_ptr(x2), _ptr(d2), None, _ptr(dx), _ptr(rstd), x2.stride(0), 0, d2.stride(0),
                          dx.stride(0), x2.shape[0], x2.shape[1], 0.0)
    with torch.cuda.device(x.device):
        _capi.check(lib.prefixlm_rmsnorm_bwd(ctypes.byref(a), _stream(x.device)), "prefixlm_rmsnorm_bwd")
    return dx.view(x.shape)


@rms_norm_bwd.register_fake
def _rms_norm_bwd_fake(x, rstd, dy):
    return x.new_empty(x.shape)


class RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, eps):
        y, rstd = rms_norm_fwd(x, eps)
        ctx.save_for_backward(x, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, rstd = ctx.saved_tensors
        return rms_norm_bwd(x, rstd, dy), None


def rms_norm(x: Tensor, eps: float = 1e-6) -> Tensor:
    """``F.rms_norm(x, (x.shape[-1],), eps=eps)`` without a weight (models/transformer.py:87)."""
    return RMSNormFunction.apply(x, eps)


# ---- projections with the norm and the SwiGLU fused in (forward only) ------------------
@torch.library.custom_op("prefixlm::proj_gemm", mutates_args=())
def proj_gemm(x: Tensor, w: Tensor, swiglu: bool, norm: bool, eps: float) -> Tensor:
    """y = rmsnorm(x) w^T, or with ``swiglu`` silu(rmsnorm(x) wg^T) * (rmsnorm(x) wu^T) for
    w = [wg; wu] (rmsnorm = identity when ``norm`` is false). x [..., K], w [N, K] bf16;
    K % 64 == 0, N % 256 == 0. Forward only: the op has no autograd formula."""
    lib = _capi.load()
    x2 = _rows(x, "x")
    if w.dtype != torch.bfloat16 or w.dim() != 2 or w.device != x.device:
        raise ValueError(f"w must be a bf16 [N, K] tensor on {x.device}")
    w2 = w if (w.stride(-1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0) else w.contiguous()
    M, K = x2.shape
    N = w2.shape[0]
    if w2.shape[1] != K:
        raise ValueError(f"w is [{N}, {w2.shape[1]}], x has K = {K}")
    nout = N // 2 if swiglu else N
    y = torch.empty((M, nout), dtype=x.dtype, device=x.device)
    rstd = torch.empty(M if norm else 0, dtype=torch.float32, device=x.device)
    a = _capi.ProjGemmArgs(_ptr(x2), _ptr(w2), _ptr(y), x2.stride(0), w2.stride(0), y.stride(0), M, K, N,
                           1 if swiglu else 0, 1 if norm else 0, float(eps), _ptr(rstd) if norm else None)
    with torch.cuda.device(x.device):
        _capi.check(lib.prefixlm_proj_gemm(ctypes.byref(a), _stream(x.device)), "prefixlm_proj_gemm")
    return y.view(*x.shape[:-1], nout)


@proj_gemm.register_fake
def _proj_gemm_fake(x, w, swiglu, norm, eps):
    n = w.shape[0] // 2 if swiglu else w.shape[0]
    return x.new_empty((*x.shape[:-1], n))


def rms_norm_linear(x: Tensor, w: Tensor, eps: float) -> Tensor:
    """F.linear(F.rms_norm(x, (K,), eps), w) in one GEMM (forward only).

    Not recommended for speed: the hand-written GEMM core runs at about 1.22 PFLOP/s on
    the config-5 shapes against 1.44 for hipBLASLt, so at 2048 -> 8192 columns the norm
    kernel plus the library GEMM is faster (0.38 vs 0.48 ms). Kept for callers that
    want the normalized activations never written."""
    return proj_gemm(x, w, False, True, float(eps))


def rms_norm_swiglu(x: Tensor, w_gate_up: Tensor, eps: float) -> Tensor:
    """silu(g) * u for [g | u] = F.linear(F.rms_norm(x, (K,), eps), w_gate_up), in one
    GEMM (forward only).

    Not recommended for speed: it saves the two elementwise passes but its GEMM core is
    slower than hipBLASLt's (about 1.22 vs 1.44 PFLOP/s), which cancels the saving inside
    the config-5 stack (150.5 vs 149.6 ms per step with and without it)."""
    return proj_gemm(x, w_gate_up, True, True, float(eps))
