"""CPU/fp32 oracle for KV-cache attention -- TEST INFRASTRUCTURE.

Only tests may import this module, as the checker; the product path never calls it.

``kvcache_attention`` restates FlashAttention's kv-cache call as the reference
uses it (``flash_attn_with_kvcache(q, k, v, k_cache, v_cache, cache_seqlens,
num_splits=1, causal)`` at models/layers.py:147-151, driven by
simple_inference_engine.py:105-112 and :179-180). FlashAttention-3 is not in the
reference tree (un-vendored, unpinned VCS install, sm90-only), so the rule below is
its documented behaviour:

* the new rows k, v [B, S, H, D] are written into the caches at rows
  len_b .. len_b + S - 1, len_b = cache_seqlens[b] (an int applies to every row);
* query i of row b attends the first lk = len_b + S cache keys (lk = len_b when
  no new rows are given); with ``causal`` only keys j <= lk - S + i (causal masks
  are aligned to the bottom-right corner when the query and key lengths differ);
* softmax scale 1/sqrt(D) unless given; fp32 softmax attention on bf16 inputs.

Pinned by (tests/test_oracle.py): a prefill (len 0, not causal) equals the varlen
oracle's bidirectional prefix segment; a decode step at position t equals row t of
the varlen oracle's forward over the same tokens with the prompt as prefix (the
rule the training op implements); causal prefill equals SDPA's is_causal path; with
a non-empty cache and S > 1 new rows, the causal call equals the last S rows of the
varlen oracle's causal segment over all len + S tokens, and the non-causal call the
last S rows of a fully bidirectional segment of len + S tokens (a diagonal that
ignores the cache length fails that check).
"""
from __future__ import annotations

import math

import torch

__all__ = ["causal_masked", "kvcache_attention"]


def causal_masked(S, lk, lk_full):
    """[1, S, lk] bool, True where query i may not see key j: j > lk_full - S + i
    (the causal diagonal aligned to the bottom-right corner of the S x lk_full score
    block, so the last query sees every key)."""
    j = torch.arange(lk).view(1, 1, lk)
    i = torch.arange(S).view(1, S, 1)
    return j > lk_full - S + i


def kvcache_attention(q, k_cache, v_cache, k=None, v=None, cache_seqlens=0, causal=False, softmax_scale=None):
    """Returns (out fp32 [B, S, H, D], new k_cache, new v_cache); the inputs are not
    modified."""
    B, S, H, D = q.shape
    Smax = k_cache.shape[1]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if isinstance(cache_seqlens, int):
        lens = [cache_seqlens] * B
    else:
        lens = [int(x) for x in cache_seqlens.tolist()]
    kc, vc = k_cache.clone(), v_cache.clone()
    if k is not None:
        for b in range(B):
            for i in range(S):
                row = lens[b] + i
                if 0 <= row < Smax:
                    kc[b, row] = k[b, i]
                    vc[b, row] = v[b, i]
    out = torch.zeros(B, S, H, D, dtype=torch.float32)
    for b in range(B):
        lk_full = lens[b] + (S if k is not None else 0)
        lk = min(Smax, lk_full)
        kk = kc[b, :lk].float().permute(1, 0, 2)            # [H, lk, D]
        vv = vc[b, :lk].float().permute(1, 0, 2)
        qq = q[b].float().permute(1, 0, 2)                  # [H, S, D]
        s = torch.matmul(qq, kk.transpose(1, 2)) * softmax_scale   # [H, S, lk]
        if causal:
            s = s.masked_fill(causal_masked(S, lk, lk_full), float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, vv).permute(1, 0, 2)
    return out, kc, vc
