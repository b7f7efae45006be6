"""KV-cache attention for inference: the reference's other FlashAttention-3 call.

``flash_attn_with_kvcache`` keeps the keyword names and the semantics of the call
at models/layers.py:147-151 (FlashAttention's kv-cache interface), as the
reference's engine drives it (simple_inference_engine.py:105-112, :179-180):

* ``k``, ``v`` [B, S, H, D] are written into ``k_cache``, ``v_cache``
  [B, Smax, H, D] in place at rows ``cache_seqlens[b] .. + S - 1`` (an int applies
  to every batch row); rows past Smax are dropped;
* query i of batch row b attends the first lk = cache_seqlens[b] + S cache keys
  (lk = cache_seqlens[b] without new rows), with ``causal`` only keys
  j <= lk - S + i (bottom-right alignment);
* ``num_splits`` is accepted and ignored: the split over keys is chosen inside
  and does not change results between calls (no atomics).

A call with ``cache_seqlens`` the int 0 (the reference's prefill) runs the
training forward kernels over the new rows; every other call runs a split-K
decode kernel that reads each cached key and value once. The op is a
``torch.library`` custom op mutating the caches, so ``torch.compile(fullgraph=True)``
traces it (simple_inference_engine.py:105, :110).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Union

import torch
from torch import Tensor

from . import _capi
from .op import _ptr, _stream

__all__ = ["flash_attn_with_kvcache", "kvcache_attn"]


def _check4(x: Tensor, name: str) -> None:
    if x.dtype != torch.bfloat16 or x.dim() != 4 or x.device.type != "cuda":
        raise ValueError(f"{name} must be a bf16 [B, S, H, D] GPU tensor (got {x.dtype} {tuple(x.shape)} on {x.device})")
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:3]) or x.data_ptr() % 16:
        raise ValueError(f"{name} needs unit stride over head_dim, strides that are multiples of 8 and a "
                         f"16-byte aligned base (got strides {x.stride()})")


@torch.library.custom_op("prefixlm::kvcache_attn", mutates_args=("k_cache", "v_cache"))
def kvcache_attn(q: Tensor, k: Optional[Tensor], v: Optional[Tensor], k_cache: Tensor, v_cache: Tensor,
                 cache_seqlens: Optional[Tensor], cache_seqlen: int, causal: bool, softmax_scale: float) -> Tensor:
    """out [B, S, H, D] bf16; k_cache / v_cache updated in place."""
    lib = _capi.load()
    B, S, H, D = q.shape
    _check4(q, "q")
    for name, x in (("k_cache", k_cache), ("v_cache", v_cache)):
        _check4(x, name)
        if x.shape[0] != B or x.shape[2] != H or x.shape[3] != D:
            raise ValueError(f"{name} must be [{B}, Smax, {H}, {D}] (got {tuple(x.shape)})")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    if (k is None) != (v is None):
        raise ValueError("k and v must be given together")
    if k is not None:
        k, v = k.contiguous() if k.data_ptr() % 16 else k, v.contiguous() if v.data_ptr() % 16 else v
        for name, x in (("k", k), ("v", v)):
            _check4(x, name)
            if tuple(x.shape) != (B, S, H, D):
                raise ValueError(f"{name} must be [{B}, {S}, {H}, {D}] (got {tuple(x.shape)})")
    dev = q.device
    if cache_seqlens is not None:
        cache_seqlens = cache_seqlens.to(device=dev, dtype=torch.int32).contiguous()
        if cache_seqlens.numel() != B:
            raise ValueError(f"cache_seqlens must hold {B} entries (got {cache_seqlens.numel()})")
    out = torch.empty((B, S, H, D), dtype=q.dtype, device=dev)
    Smax = k_cache.shape[1]
    ws_bytes = lib.prefixlm_kvcache_workspace_size(B, S, H, D, Smax)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    z = (0, 0, 0)
    ks = k.stride()[:3] if k is not None else z
    vs = v.stride()[:3] if v is not None else z
    a = _capi.KvcacheArgs(
        _ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(out),
        *q.stride()[:3], *ks, *vs, *k_cache.stride()[:3], *v_cache.stride()[:3], *out.stride()[:3],
        _ptr(cache_seqlens), int(cache_seqlen), B, S, H, D, Smax, 1 if causal else 0, float(softmax_scale),
        _ptr(ws), ws_bytes)
    with torch.cuda.device(dev):
        _capi.check(lib.prefixlm_kvcache_fwd(ctypes.byref(a), _stream(dev)), "prefixlm_kvcache_fwd")
    return out


@kvcache_attn.register_fake
def _kvcache_attn_fake(q, k, v, k_cache, v_cache, cache_seqlens, cache_seqlen, causal, softmax_scale):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


def flash_attn_with_kvcache(q: Tensor, k_cache: Tensor, v_cache: Tensor, k: Optional[Tensor] = None,
                            v: Optional[Tensor] = None, cache_seqlens: Union[int, Tensor, None] = None,
                            softmax_scale: Optional[float] = None, causal: bool = False,
                            num_splits: int = 0, **unsupported) -> Tensor:
    """Drop-in for the reference's kv-cache call (models/layers.py:148-151).

    q [B, S, H, 128] bf16; k_cache, v_cache [B, Smax, H, 128] bf16 (updated in place);
    k, v [B, S, H, 128] or None; cache_seqlens int or int32 [B] tensor (None = 0).
    Options of FlashAttention's interface that the reference does not use (rotary,
    paged or indexed caches, windows, softcap, returning the LSE, ...) raise."""
    used = {n: x for n, x in unsupported.items() if x not in (None, False, 0, 0.0, (-1, -1))}
    if used:
        raise NotImplementedError(f"flash_attn_with_kvcache: unsupported arguments {sorted(used)}")
    del num_splits
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    if cache_seqlens is None:
        cache_seqlens = 0
    if isinstance(cache_seqlens, int):
        return kvcache_attn(q, k, v, k_cache, v_cache, None, cache_seqlens, bool(causal), float(softmax_scale))
    return kvcache_attn(q, k, v, k_cache, v_cache, cache_seqlens, 0, bool(causal), float(softmax_scale))
