"""The attention layer's prologue and epilogue fused around the PrefixLM kernels.

The reference's ``Attention.forward`` (models/layers.py:129-155) splits the fused
gate/q/k/v projection into heads (:131-135), applies fp32 RoPE to q and k
(:23-38, :138-140), calls the attention op (:145) and gates its output with
``sigmoid(gate)`` (:154). As separate PyTorch ops that is several passes over
[T, H, D] tensors per call, forward and backward, plus the copies autograd makes
to assemble the projection's gradient from its four slices.

``fused_attention_layer`` runs the same computation as:

* one RoPE kernel reading q and k straight from the projection output and writing
  the rotated pair (bitwise the reference's fp32 RoPE);
* the attention forward, whose epilogue also writes ``sigmoid(gate) * O``;
* in the backward, the attention pre-pass also computes the gate's gradient and
  ``dO = dy * sigmoid(gate)``; dQ, dK, dV and dgate are written directly into
  their slices of the projection's gradient, and one in-place kernel applies the
  transposed rotation to the dQ and dK slices.

Rounding: RoPE and the gated output match the reference's bf16 results; the
gradients of the gate and of the RoPE inputs are each rounded once where autograd
rounds twice.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _capi
from .op import (_as_cpu_scalar_tensor, _check_lists_after_launch, _check_plan_before_launch, _check_q_amax,
                 _cpu_scalar, _ds_arg, _ds_blocks_arg, _meta, _plan_arg, _ptr, _q_amax_count, _stream)

__all__ = ["fused_attention_layer", "FusedAttentionLayer", "rope", "attn_layer_fwd", "attn_layer_bwd"]

D_HEAD = 128


def _check_gqkv(gqkv: Tensor) -> Tuple[int, int, int]:
    if gqkv.dtype != torch.bfloat16 or gqkv.dim() != 3 or gqkv.device.type != "cuda":
        raise ValueError(f"gqkv must be a bf16 [T, 4H, D] GPU tensor (got {gqkv.dtype} {tuple(gqkv.shape)} "
                         f"on {gqkv.device})")
    T, H4, D = gqkv.shape
    if H4 % 4 or D != D_HEAD:
        raise ValueError(f"gqkv must be [T, 4H, 128] (gate, q, k, v heads), got {tuple(gqkv.shape)}")
    return T, H4 // 4, D


def _check_cos_sin(cos: Tensor, sin: Tensor, T: int) -> Tuple[Tensor, Tensor]:
    out = []
    for name, x in (("cos", cos), ("sin", sin)):
        if x.dtype != torch.float32 or tuple(x.shape) != (T, D_HEAD):
            raise ValueError(f"{name} must be float32 [{T}, {D_HEAD}] (got {x.dtype} {tuple(x.shape)})")
        if x.stride(-1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
            x = x.contiguous()
        out.append(x)
    return out[0], out[1]


def rope(x: Tensor, y: Tensor, cos: Tensor, sin: Tensor, backward: bool = False) -> None:
    """y = rope(x) (or its transpose) for bf16 [T, heads, 128] views; y may be x."""
    lib = _capi.load()
    a = _capi.RopeArgs(_ptr(x), _ptr(y), _ptr(cos), _ptr(sin), x.stride(0), x.stride(1), y.stride(0),
                       y.stride(1), cos.stride(0), x.shape[0], x.shape[1], x.shape[2], 1 if backward else 0)
    with torch.cuda.device(x.device):
        _capi.check(lib.prefixlm_rope(ctypes.byref(a), _stream(x.device)), "prefixlm_rope")


def _scalars(total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all):
    return [_cpu_scalar(x, n) for x, n in ((total_seqlen, "total_seqlen"), (numseqs, "numseqs"),
                                           (max_seqlen_prefix, "max_seqlen_prefix"),
                                           (max_seqlen_causal, "max_seqlen_causal"),
                                           (max_seqlen_all, "max_seqlen_all"))]


@torch.library.custom_op("prefixlm::attn_layer_fwd", mutates_args=())
def attn_layer_fwd(gqkv: Tensor, cos: Tensor, sin: Tensor, is_causal: bool,
                   prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
                   total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
                   max_seqlen_causal: Tensor, max_seqlen_all: Tensor, softmax_scale: float,
                   plan: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(y, qk, out, lse, out_lo, q_amax): y = sigmoid(gate) * attention [T, H, D], the
    rotated q/k pair qk [T, 2H, D] and the attention's out, lse, out_lo, q_amax (saved for
    the backward)."""
    lib = _capi.load()
    T, H, D = _check_gqkv(gqkv)
    gqkv = gqkv.contiguous()
    dev = gqkv.device
    total, nseq, mp, mc, ma = _scalars(total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all)
    cos, sin = _check_cos_sin(cos, sin, T)
    pre, cau, cu = (_meta(t, dev) for t in (prefix_lens, causal_lens, cu_seqlens))
    qk = torch.empty((T, 2 * H, D), dtype=gqkv.dtype, device=dev)
    rope(gqkv[:, H:3 * H], qk, cos, sin)
    q, k, v, gate = qk[:, :H], qk[:, H:], gqkv[:, 3 * H:], gqkv[:, :H]
    out = torch.empty((T, H, D), dtype=gqkv.dtype, device=dev)
    out_lo = torch.empty((T, H, D), dtype=torch.int8, device=dev)
    y = torch.empty_like(out)
    lse = torch.empty((H, T), dtype=torch.float32, device=dev)
    q_amax = torch.empty(_q_amax_count(T, H), dtype=torch.float32, device=dev)
    plan_p, plan_b, plan = _plan_arg(plan, dev)
    _check_plan_before_launch(plan, (pre, cau, cu, total, nseq, is_causal))
    ws_bytes = 0 if plan is not None else lib.prefixlm_fwd_workspace_size(T, H, D, total, nseq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    a = _capi.FwdArgs(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(out_lo), _ptr(lse),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), out_lo.stride(0), out_lo.stride(1),
        _ptr(pre), _ptr(cau), _ptr(cu), min(pre.numel(), cau.numel(), cu.numel()),
        T, H, D, total, nseq, mp, mc, ma, 1 if is_causal else 0, float(softmax_scale),
        _ptr(ws), ws_bytes, plan_p, plan_b,
        _ptr(gate), _ptr(y), gate.stride(0), gate.stride(1), y.stride(0), y.stride(1),
        _capi.active_timer(), _ptr(q_amax))
    with torch.cuda.device(dev):
        _capi.check(lib.prefixlm_fwd(ctypes.byref(a), _stream(dev)), "prefixlm_fwd (gated)")
        _check_lists_after_launch(lib, ws, dev, plan)
    return y, qk, out, lse, out_lo, q_amax


@attn_layer_fwd.register_fake
def _attn_layer_fwd_fake(gqkv, cos, sin, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                         numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, softmax_scale,
                         plan=None):
    T, H4, D = gqkv.shape
    H = H4 // 4
    mk = lambda *s, dt=gqkv.dtype: torch.empty(s, dtype=dt, device=gqkv.device)  # noqa: E731
    return (mk(T, H, D), mk(T, 2 * H, D), mk(T, H, D), mk(H, T, dt=torch.float32), mk(T, H, D, dt=torch.int8),
            mk(_q_amax_count(T, H), dt=torch.float32))


@torch.library.custom_op("prefixlm::attn_layer_bwd", mutates_args=())
def attn_layer_bwd(dy: Tensor, gqkv: Tensor, qk: Tensor, out: Tensor, lse: Tensor, out_lo: Tensor,
                   q_amax: Tensor, cos: Tensor, sin: Tensor, is_causal: bool,
                   prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
                   total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
                   max_seqlen_causal: Tensor, max_seqlen_all: Tensor, softmax_scale: float,
                   plan: Optional[Tensor] = None, plan_ds_blocks: Optional[Tensor] = None) -> Tensor:
    """Gradient of the projection output gqkv [T, 4H, D] (gate, q, k, v slices)."""
    lib = _capi.load()
    T, H, D = _check_gqkv(gqkv)
    gqkv = gqkv.contiguous()
    dev = gqkv.device
    total, nseq, mp, mc, ma = _scalars(total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all)
    cos, sin = _check_cos_sin(cos, sin, T)
    dy = dy.contiguous()
    q_amax = _check_q_amax(q_amax, T, H, dev)
    pre, cau, cu = (_meta(t, dev) for t in (prefix_lens, causal_lens, cu_seqlens))
    q, k, v, gate = qk[:, :H], qk[:, H:], gqkv[:, 3 * H:], gqkv[:, :H]
    dg = torch.empty_like(gqkv)
    dgate, dq, dk, dv = dg[:, :H], dg[:, H:2 * H], dg[:, 2 * H:3 * H], dg[:, 3 * H:]
    dout_attn = torch.empty((T, H, D), dtype=gqkv.dtype, device=dev)
    ws_bytes = lib.prefixlm_bwd_workspace_size(T, H, D, total, nseq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    plan_p, plan_b, plan = _plan_arg(plan, dev)
    dsb = _ds_blocks_arg(plan_ds_blocks) if plan is not None else 0
    _check_plan_before_launch(plan, (pre, cau, cu, total, nseq, is_causal), dsb)
    ds_p, ds_b, ds_buf, dsb = _ds_arg(lib, T, H, nseq, ma, dev, dsb)
    a = _capi.BwdArgs(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(out_lo), _ptr(dy), _ptr(lse), _ptr(q_amax),
        _ptr(dq), _ptr(dk), _ptr(dv),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), out_lo.stride(0), out_lo.stride(1),
        dy.stride(0), dy.stride(1),
        dq.stride(0), dq.stride(1), dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1),
        _ptr(pre), _ptr(cau), _ptr(cu), min(pre.numel(), cau.numel(), cu.numel()),
        T, H, D, total, nseq, mp, mc, ma, 1 if is_causal else 0, float(softmax_scale),
        _ptr(ws), ws_bytes, plan_p, plan_b,
        _ptr(gate), _ptr(dgate), _ptr(dout_attn),
        gate.stride(0), gate.stride(1), dgate.stride(0), dgate.stride(1),
        dout_attn.stride(0), dout_attn.stride(1), _capi.active_timer(), ds_p, ds_b, dsb)
    with torch.cuda.device(dev):
        _capi.check(lib.prefixlm_bwd(ctypes.byref(a), _stream(dev)), "prefixlm_bwd (gated)")
        _check_lists_after_launch(lib, ws, dev, plan)
    dqk = dg[:, H:3 * H]
    rope(dqk, dqk, cos, sin, backward=True)
    return dg


@attn_layer_bwd.register_fake
def _attn_layer_bwd_fake(dy, gqkv, qk, out, lse, out_lo, q_amax, cos, sin, is_causal, prefix_lens, causal_lens,
                         cu_seqlens, total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal,
                         max_seqlen_all, softmax_scale, plan=None, plan_ds_blocks=None):
    return torch.empty(gqkv.shape, dtype=gqkv.dtype, device=gqkv.device)


class FusedAttentionLayer(torch.autograd.Function):
    """autograd glue of the fused layer; saves the projection output, the rotated q/k,
    out, lse, out_lo, q_amax and the metadata (cos/sin get no gradient, as the reference's
    non-persistent RotaryEmbedding buffers, models/layers.py:49-50)."""

    @staticmethod
    def forward(ctx, gqkv, cos, sin, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, softmax_scale, plan=None,
                plan_ds_blocks=None):
        y, qk, out, lse, out_lo, q_amax = attn_layer_fwd(gqkv, cos, sin, is_causal, prefix_lens, causal_lens,
                                                         cu_seqlens, total_seqlen, numseqs, max_seqlen_prefix,
                                                         max_seqlen_causal, max_seqlen_all, softmax_scale, plan)
        ctx.save_for_backward(gqkv, qk, out, lse, out_lo, q_amax, cos, sin, prefix_lens, causal_lens, cu_seqlens,
                              total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, plan,
                              plan_ds_blocks)
        ctx.is_causal = is_causal
        ctx.softmax_scale = softmax_scale
        return y

    @staticmethod
    def backward(ctx, dy):
        (gqkv, qk, out, lse, out_lo, q_amax, cos, sin, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
         numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, plan, plan_ds_blocks) = ctx.saved_tensors
        dg = attn_layer_bwd(dy, gqkv, qk, out, lse, out_lo, q_amax, cos, sin, ctx.is_causal, prefix_lens,
                            causal_lens, cu_seqlens, total_seqlen, numseqs, max_seqlen_prefix,
                            max_seqlen_causal, max_seqlen_all, ctx.softmax_scale, plan, plan_ds_blocks)
        return dg, *((None,) * 14)


def fused_attention_layer(gqkv: Tensor, cos: Tensor, sin: Tensor, is_causal: bool,
                          prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
                          total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
                          max_seqlen_causal: Tensor, max_seqlen_all: Tensor,
                          softmax_scale: Optional[float] = None, plan: Optional[Tensor] = None,
                          plan_ds_blocks: Optional[Tensor] = None) -> Tensor:
    """sigmoid(gate) * attention(rope(q), rope(k), v) for the projection output
    gqkv [T, 4H, 128] bf16 (heads ordered gate, q, k, v as split at
    models/layers.py:135) and the gathered cos, sin [T, 128] fp32. Returns
    [T, H, 128] bf16; reshape to [T, H*128] for the output projection. ``plan`` and
    ``plan_ds_blocks`` as in ``flash_attn_varlen_prefixlm``."""
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(gqkv.shape[-1])
    scal = [_as_cpu_scalar_tensor(x) for x in
            (total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all)]
    if plan_ds_blocks is not None:
        plan_ds_blocks = _as_cpu_scalar_tensor(plan_ds_blocks)
    return FusedAttentionLayer.apply(gqkv, cos, sin, bool(is_causal), prefix_lens, causal_lens, cu_seqlens,
                                     *scal, float(softmax_scale), plan, plan_ds_blocks)
