"""PyTorch operators for packed varlen PrefixLM attention on MI355X.

Mirrors the operator layer of the reference wrapper
(models/flash_attention_prefixlm_v2.py:88-282):

* ``prefixlm::varlen_fwd`` / ``prefixlm::varlen_bwd`` are ``torch.library``
  custom ops with fake (meta) implementations, so a ``torch.compile(dynamic=False)``
  step treats them as opaque, shape-static calls (reference :88, :134, :152, :215);
* ``FlashAttnVarlenPrefixLM`` is the ``autograd.Function`` joining them
  (reference :234-268);
* ``flash_attn_varlen_prefixlm`` is the public entry with the reference signature
  (reference :271-282) plus an optional trailing ``softmax_scale`` (default
  ``1/sqrt(head_dim)``, the value FA3 uses when the reference passes None, :73).

Differences a caller can observe: the forward op returns one merged LSE [H, T]
instead of two half-valid ones (every valid row belongs to exactly one of the
reference's two passes); the outputs are always contiguous.

The scalar metadata must be CPU tensors, as in the reference (asserted at :103 and
:169), so the op never synchronizes with the device to learn its launch sizes.
Set ``PREFIXLM_CHECK_METADATA=1`` to make every call synchronize and raise if the
kernels saw inconsistent segment metadata (or, with a plan, if the plan differs from
the one the metadata gives).

An optional ``plan`` (``prefixlm.plan.build_plan``, int32, on the device with the
rest of the batch) replaces the per-call work-list kernel; with it, the optional CPU
scalar ``plan_ds_blocks`` (``prefixlm.plan.plan_ds_blocks`` of the same plan; both come
from ``prefixlm.plan.plan_inputs``) sizes the backward's dS buffer to exactly the blocks
the batch attends instead of the bound the max_seqlen scalars give.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _capi

__all__ = ["flash_attn_varlen_prefixlm", "FlashAttnVarlenPrefixLM", "varlen_fwd", "varlen_bwd"]

_CHECK_METADATA = os.environ.get("PREFIXLM_CHECK_METADATA", "0") not in ("", "0")


def _cpu_scalar(x, name) -> int:
    if isinstance(x, Tensor):
        assert x.device.type == "cpu", f"{name} must be a CPU tensor (got {x.device})"
        return int(x.item())
    return int(x)


def _as_kernel_operand(x: Tensor, name: str) -> Tensor:
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (got {x.dtype})")
    if x.dim() != 3:
        raise ValueError(f"{name} must be [tokens, heads, head_dim] (got shape {tuple(x.shape)})")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU (got {x.device})")
    # the kernels read 16-byte vectors: unit stride over head_dim, 8-element
    # multiples over tokens and heads, 16-byte aligned base
    if (x.stride(-1) != 1 or x.stride(0) % 8 or x.stride(1) % 8 or x.stride(0) < x.shape[-1]
            or x.data_ptr() % 16):
        x = x.contiguous()
    return x


def _as_residual_operand(x: Tensor, like: Tensor) -> Tensor:
    """out_lo: int8 codes shaped like out, with 16-byte rows and strides."""
    if x.dtype != torch.int8:
        raise TypeError(f"out_lo must be int8 (got {x.dtype})")
    if tuple(x.shape) != tuple(like.shape) or x.device != like.device:
        raise ValueError(f"out_lo must be {tuple(like.shape)} on {like.device} (got {tuple(x.shape)} on {x.device})")
    if x.stride(-1) != 1 or x.stride(0) % 16 or x.stride(1) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _meta(x: Tensor, device) -> Tensor:
    if x.dtype != torch.int32 or x.device != device or not x.is_contiguous():
        x = x.to(device=device, dtype=torch.int32).contiguous()
    return x


def _ptr(x: Optional[Tensor]):
    return ctypes.c_void_p(x.data_ptr()) if x is not None else ctypes.c_void_p(0)


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# Largest dS buffer the backward allocates to compute dQ from the stored dS: the
# PREFIXLM_DS_MAX_BYTES environment variable, else an eighth of the device's memory.
# Batches that need more (or PREFIXLM_DS_MAX_BYTES=0), and calls whose allocation fails,
# recompute S, P and dP in the dQ kernel instead. The buffer holds 2 bytes per attended
# (query, key) pair and head, rounded up to blocks of 32 x 64 (exact with plan_ds_blocks;
# without it, the bound of about 2 * heads * tokens * max_seqlen_all bytes).
_DEV_MEM = {}


def _ds_cap(dev) -> int:
    env = os.environ.get("PREFIXLM_DS_MAX_BYTES")
    if env is not None:
        return int(env)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _DEV_MEM:
        _DEV_MEM[idx] = torch.cuda.get_device_properties(idx).total_memory
    return _DEV_MEM[idx] // 8


def _ds_bytes(lib, T, H, nseq, max_seqlen_all, ds_blocks: int, dev) -> int:
    """Bytes of the dS buffer the backward of such a batch gets (0: dQ is recomputed);
    ds_blocks > 0: blocks per head (a plan's exact count), else the scalars' bound."""
    if ds_blocks > 0:
        n = lib.prefixlm_bwd_ds_bytes_blocks(T, H, nseq, ds_blocks) if max_seqlen_all <= 32768 else 0
    else:
        n = lib.prefixlm_bwd_ds_bytes(T, H, nseq, max_seqlen_all)
    return n if 0 < n <= _ds_cap(dev) else 0


def _ds_blocks_arg(plan_ds_blocks) -> int:
    if plan_ds_blocks is None:
        return 0
    n = _cpu_scalar(plan_ds_blocks, "plan_ds_blocks")
    if n < 0:
        raise ValueError(f"plan_ds_blocks={n} < 0")
    return n


def ds_path_used(T, H, nseq, max_seqlen_all, plan_ds_blocks=None, device=None) -> bool:
    """Whether the backward of a batch of this shape computes dQ from the stored dS
    (unless its allocation fails)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    return _ds_bytes(_capi.load(), T, H, nseq, max_seqlen_all, _ds_blocks_arg(plan_ds_blocks), dev) > 0


def ds_buffer_bytes(T, H, nseq, max_seqlen_all, plan_ds_blocks=None, device=None) -> int:
    """Bytes of the dS buffer the backward of such a batch allocates (0: none)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    return _ds_bytes(_capi.load(), T, H, nseq, max_seqlen_all, _ds_blocks_arg(plan_ds_blocks), dev)


def _ds_arg(lib, T, H, nseq, max_seqlen_all, dev, ds_blocks: int = 0):
    """(pointer, bytes, tensor, blocks per head) of the optional dS buffer of
    prefixlm_bwd; no buffer when it would exceed the cap or its allocation fails."""
    n = _ds_bytes(lib, T, H, nseq, max_seqlen_all, ds_blocks, dev)
    if n == 0:
        return ctypes.c_void_p(0), 0, None, 0
    try:
        buf = torch.empty(n, dtype=torch.uint8, device=dev)
    except torch.OutOfMemoryError:
        return ctypes.c_void_p(0), 0, None, 0
    return _ptr(buf), n, buf, ds_blocks


def _q_amax_count(T: int, H: int) -> int:
    """Slots of the forward's max |q| output (a function of the shape only)."""
    return int(_capi.load().prefixlm_fwd_q_amax_count(T, H))


def _check_q_amax(x: Tensor, T: int, H: int, device) -> Tensor:
    n = _q_amax_count(T, H)
    if x.dtype != torch.float32 or x.dim() != 1 or x.numel() != n or x.device != device:
        raise ValueError(f"q_amax must be the forward's float32 [{n}] on {device} "
                         f"(got {x.dtype} {tuple(x.shape)} on {x.device})")
    return x.contiguous()


def _plan_arg(plan: Optional[Tensor], device):
    """(pointer, bytes, tensor kept alive) for an optional plan."""
    if plan is None:
        return ctypes.c_void_p(0), 0, None
    if plan.dtype != torch.int32 or plan.dim() != 1:
        raise TypeError(f"plan must be a 1-D int32 tensor (got {plan.dtype} {tuple(plan.shape)})")
    if plan.device != device or not plan.is_contiguous() or plan.data_ptr() % 256:
        plan = plan.to(device=device, non_blocking=True).contiguous().clone()
    return _ptr(plan), plan.numel() * 4, plan


def _check_plan(plan: Tensor, pre: Tensor, cau: Tensor, cu: Tensor, total: int, nseq: int,
                is_causal: bool, ds_blocks: int = 0):
    from .plan import build_plan, plan_ds_blocks
    want = build_plan({"prefix_lens": pre, "causal_lens": cau, "cu_seqlens": cu},
                      {"numseqs": nseq, "total_seqlen": total}, is_causal)
    got = plan.detach().cpu().numpy()
    import numpy as np
    # the item order only affects speed: compare each list's header and item set
    if got.shape != want.shape or not np.array_equal(np.sort(got), np.sort(want)):
        raise RuntimeError("prefixlm plan does not match the batch metadata")
    if ds_blocks and ds_blocks < plan_ds_blocks(want):
        raise RuntimeError(f"plan_ds_blocks={ds_blocks} is below the plan's {plan_ds_blocks(want)} blocks")


def _check_plan_before_launch(plan: Optional[Tensor], meta, ds_blocks: int = 0):
    """Checking mode: a caller's plan is compared with the one the call's metadata
    gives before any kernel is launched with it."""
    if _CHECK_METADATA and plan is not None:
        _check_plan(plan, *meta, ds_blocks=ds_blocks)


def _check_lists_after_launch(lib, ws: Optional[Tensor], device, plan=None):
    """Checking mode: device-built work lists carry an error word the list kernel
    wrote; reading it synchronizes with the stream."""
    if _CHECK_METADATA and plan is None:
        err = ctypes.c_int32(0)
        _capi.check(lib.prefixlm_check_workspace(_ptr(ws), _stream(device), ctypes.byref(err)),
                    "prefixlm metadata check")


@torch.library.custom_op("prefixlm::varlen_fwd", mutates_args=())
def varlen_fwd(q: Tensor, k: Tensor, v: Tensor, is_causal: bool,
               prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
               total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
               max_seqlen_causal: Tensor, max_seqlen_all: Tensor,
               softmax_scale: float, plan: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """out [T,H,D] bf16, merged lse [H,T] fp32, out_lo [T,H,D] int8, the rounding
    residual of out (in 1/256 of out's bf16 ulp) that the backward uses for a precise
    rowsum(dO * O), and q_amax (fp32, one max |q| per workgroup of the kernel's grid)
    from which the backward scales q to fp16 (reference op :88-131)."""
    lib = _capi.load()
    total = _cpu_scalar(total_seqlen, "total_seqlen")
    nseq = _cpu_scalar(numseqs, "numseqs")
    mp = _cpu_scalar(max_seqlen_prefix, "max_seqlen_prefix")
    mc = _cpu_scalar(max_seqlen_causal, "max_seqlen_causal")
    ma = _cpu_scalar(max_seqlen_all, "max_seqlen_all")
    q = _as_kernel_operand(q, "q")
    k = _as_kernel_operand(k, "k")
    v = _as_kernel_operand(v, "v")
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    T, H, D = q.shape
    dev = q.device
    pre, cau, cu = (_meta(t, dev) for t in (prefix_lens, causal_lens, cu_seqlens))
    out = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    out_lo = torch.empty((T, H, D), dtype=torch.int8, device=dev)
    lse = torch.empty((H, T), dtype=torch.float32, device=dev)
    q_amax = torch.empty(_q_amax_count(T, H), dtype=torch.float32, device=dev)
    plan_p, plan_b, plan = _plan_arg(plan, dev)
    _check_plan_before_launch(plan, (pre, cau, cu, total, nseq, is_causal))
    # the workspace holds the work list: none with a plan
    ws_bytes = 0 if plan is not None else lib.prefixlm_fwd_workspace_size(T, H, D, total, nseq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    a = _capi.FwdArgs(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(out_lo), _ptr(lse),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), out_lo.stride(0), out_lo.stride(1),
        _ptr(pre), _ptr(cau), _ptr(cu), min(pre.numel(), cau.numel(), cu.numel()),
        T, H, D, total, nseq, mp, mc, ma, 1 if is_causal else 0, float(softmax_scale),
        _ptr(ws), ws_bytes, plan_p, plan_b,
        timer=_capi.active_timer(), q_amax=_ptr(q_amax))
    with torch.cuda.device(dev):
        _capi.check(lib.prefixlm_fwd(ctypes.byref(a), _stream(dev)), "prefixlm_fwd")
        _check_lists_after_launch(lib, ws, dev, plan)
    return out, lse, out_lo, q_amax


@varlen_fwd.register_fake
def _varlen_fwd_fake(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                     numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, softmax_scale,
                     plan=None):
    T, H, _ = q.shape
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((H, T), dtype=torch.float32, device=q.device)
    out_lo = torch.empty(q.shape, dtype=torch.int8, device=q.device)
    q_amax = torch.empty(_q_amax_count(T, H), dtype=torch.float32, device=q.device)
    return out, lse, out_lo, q_amax


@torch.library.custom_op("prefixlm::varlen_bwd", mutates_args=())
def varlen_bwd(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, dout: Tensor, out: Tensor,
               lse: Tensor, out_lo: Tensor, q_amax: Tensor, prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
               total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
               max_seqlen_causal: Tensor, max_seqlen_all: Tensor,
               softmax_scale: float, plan: Optional[Tensor] = None,
               plan_ds_blocks: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """dq, dk, dv [T,H,D] bf16 (reference op :152-212)."""
    lib = _capi.load()
    total = _cpu_scalar(total_seqlen, "total_seqlen")
    nseq = _cpu_scalar(numseqs, "numseqs")
    mp = _cpu_scalar(max_seqlen_prefix, "max_seqlen_prefix")
    mc = _cpu_scalar(max_seqlen_causal, "max_seqlen_causal")
    ma = _cpu_scalar(max_seqlen_all, "max_seqlen_all")
    q = _as_kernel_operand(q, "q")
    k = _as_kernel_operand(k, "k")
    v = _as_kernel_operand(v, "v")
    dout = _as_kernel_operand(dout, "dout")
    out = _as_kernel_operand(out, "out")
    out_lo = _as_residual_operand(out_lo, out)
    T, H, D = q.shape
    dev = q.device
    if lse.dtype != torch.float32 or tuple(lse.shape) != (H, T):
        raise ValueError(f"lse must be float32 [{H}, {T}] (got {lse.dtype} {tuple(lse.shape)})")
    lse = lse.contiguous()
    q_amax = _check_q_amax(q_amax, T, H, dev)
    pre, cau, cu = (_meta(t, dev) for t in (prefix_lens, causal_lens, cu_seqlens))
    dq = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    dk = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    dv = torch.empty((T, H, D), dtype=q.dtype, device=dev)
    ws_bytes = lib.prefixlm_bwd_workspace_size(T, H, D, total, nseq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    plan_p, plan_b, plan = _plan_arg(plan, dev)
    dsb = _ds_blocks_arg(plan_ds_blocks) if plan is not None else 0
    _check_plan_before_launch(plan, (pre, cau, cu, total, nseq, is_causal), dsb)
    ds_p, ds_b, ds_buf, dsb = _ds_arg(lib, T, H, nseq, ma, dev, dsb)
    a = _capi.BwdArgs(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(out_lo), _ptr(dout), _ptr(lse), _ptr(q_amax),
        _ptr(dq), _ptr(dk), _ptr(dv),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), out_lo.stride(0), out_lo.stride(1),
        dout.stride(0), dout.stride(1),
        dq.stride(0), dq.stride(1), dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1),
        _ptr(pre), _ptr(cau), _ptr(cu), min(pre.numel(), cau.numel(), cu.numel()),
        T, H, D, total, nseq, mp, mc, ma, 1 if is_causal else 0, float(softmax_scale),
        _ptr(ws), ws_bytes, plan_p, plan_b,
        timer=_capi.active_timer(), ds_buf=ds_p, ds_buf_bytes=ds_b, ds_blocks=dsb)
    with torch.cuda.device(dev):
        _capi.check(lib.prefixlm_bwd(ctypes.byref(a), _stream(dev)), "prefixlm_bwd")
        _check_lists_after_launch(lib, ws, dev, plan)
    return dq, dk, dv


@varlen_bwd.register_fake
def _varlen_bwd_fake(q, k, v, is_causal, dout, out, lse, out_lo, q_amax, prefix_lens, causal_lens, cu_seqlens,
                     total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all,
                     softmax_scale, plan=None, plan_ds_blocks=None):
    return (torch.empty(q.shape, dtype=q.dtype, device=q.device),
            torch.empty(k.shape, dtype=k.dtype, device=k.device),
            torch.empty(v.shape, dtype=v.dtype, device=v.device))


class FlashAttnVarlenPrefixLM(torch.autograd.Function):
    """autograd glue (reference :234-268); saves q, k, v, out, lse, out_lo, q_amax and the
    metadata."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens,
                total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all,
                softmax_scale, plan=None, plan_ds_blocks=None):
        out, lse, out_lo, q_amax = varlen_fwd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens,
                                              total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal,
                                              max_seqlen_all, softmax_scale, plan)
        ctx.save_for_backward(q, k, v, out, lse, out_lo, q_amax, prefix_lens, causal_lens, cu_seqlens,
                              total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal,
                              max_seqlen_all, plan, plan_ds_blocks)
        ctx.is_causal = is_causal
        ctx.softmax_scale = softmax_scale
        return out

    @staticmethod
    def backward(ctx, dout):
        (q, k, v, out, lse, out_lo, q_amax, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
         max_seqlen_prefix, max_seqlen_causal, max_seqlen_all, plan, plan_ds_blocks) = ctx.saved_tensors
        dq, dk, dv = varlen_bwd(q, k, v, ctx.is_causal, dout, out, lse, out_lo, q_amax, prefix_lens, causal_lens,
                                cu_seqlens, total_seqlen, numseqs, max_seqlen_prefix,
                                max_seqlen_causal, max_seqlen_all, ctx.softmax_scale, plan, plan_ds_blocks)
        return dq, dk, dv, *((None,) * 12)


def _as_cpu_scalar_tensor(x) -> Tensor:
    if isinstance(x, Tensor):
        return x
    return torch.tensor(int(x), dtype=torch.int64)


def flash_attn_varlen_prefixlm(q: Tensor, k: Tensor, v: Tensor, is_causal: bool,
                               prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
                               total_seqlen: Tensor, numseqs: Tensor, max_seqlen_prefix: Tensor,
                               max_seqlen_causal: Tensor, max_seqlen_all: Tensor,
                               softmax_scale: Optional[float] = None,
                               plan: Optional[Tensor] = None,
                               plan_ds_blocks: Optional[Tensor] = None) -> Tensor:
    """Packed varlen PrefixLM attention, drop-in for the reference entry point
    (models/flash_attention_prefixlm_v2.py:271-282).

    q, k, v: bf16 [T, H, D] on the GPU (D = 128); prefix_lens / causal_lens /
    cu_seqlens: int32 [T] device tensors in the ``compute_aux_seq_tensors_scalars``
    format; the five scalars: 0-d int64 CPU tensors. Returns out [T, H, D].
    ``plan`` (optional, not in the reference): the batch's work-list plan from
    ``prefixlm.plan.build_plan``, int32 on the device; the calls then skip their
    work-list kernel. ``plan_ds_blocks`` (optional, with ``plan``): that plan's
    ``prefixlm.plan.plan_ds_blocks`` as a CPU scalar, which sizes the backward's dS
    buffer exactly (``prefixlm.plan.plan_inputs`` returns both).
    """
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    scal = [_as_cpu_scalar_tensor(x) for x in
            (total_seqlen, numseqs, max_seqlen_prefix, max_seqlen_causal, max_seqlen_all)]
    if plan_ds_blocks is not None:
        plan_ds_blocks = _as_cpu_scalar_tensor(plan_ds_blocks)
    return FlashAttnVarlenPrefixLM.apply(q, k, v, bool(is_causal), prefix_lens, causal_lens,
                                         cu_seqlens, *scal, float(softmax_scale), plan, plan_ds_blocks)
