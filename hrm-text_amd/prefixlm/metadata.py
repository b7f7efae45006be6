"""Packed-batch metadata for PrefixLM attention (host side, numpy).

`compute_aux_seq_tensors_scalars` keeps the name, arguments and outputs of the
reference helper (models/flash_attention_prefixlm_v2.py:10-24, called from
dataset_new.py:130-131), so a data loader that imports it keeps working:

* ``prefix_lens`` / ``causal_lens`` are zero-padded to ``batch_max_tokens``;
* ``cu_seqlens`` is ``[0, cumsum(prefix+causal)...]`` and then zero-padded,
  i.e. the tail after the last boundary is 0, not the total (reference :16);
* the scalars are ``total_seqlen, numseqs, max_seqlen_prefix,
  max_seqlen_causal, max_seqlen_all`` as Python ints (reference :19-23).

The rest of the module is this build's own arithmetic on the same metadata:
the count of attended (query, key) pairs that defines "useful FLOPs", and the
per-segment tile counts used to size kernel grids.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "compute_aux_seq_tensors_scalars",
    "useful_entries",
    "useful_flops",
    "SCALAR_NAMES",
    "TENSOR_NAMES",
]

# Keyword names the attention entry point receives (reference :271-278).
TENSOR_NAMES = ("prefix_lens", "causal_lens", "cu_seqlens")
SCALAR_NAMES = ("total_seqlen", "numseqs", "max_seqlen_prefix",
                "max_seqlen_causal", "max_seqlen_all")


def compute_aux_seq_tensors_scalars(prefix_lens: np.ndarray, causal_lens: np.ndarray,
                                    batch_max_tokens: int):
    """Pad per-segment lengths to a fixed token count and derive the scalars.

    Mirrors models/flash_attention_prefixlm_v2.py:10-24. ``prefix_lens`` and
    ``causal_lens`` are 1-D integer arrays of equal length ``nseq``; the result
    tensors have length ``batch_max_tokens`` and keep the input dtype (int32 in
    the reference data loader, dataset_new.py:130).
    """
    prefix_lens = np.asarray(prefix_lens)
    causal_lens = np.asarray(causal_lens)
    if prefix_lens.ndim != 1 or prefix_lens.shape != causal_lens.shape:
        raise ValueError("prefix_lens and causal_lens must be 1-D arrays of equal length")
    nseq = int(prefix_lens.shape[0])
    if nseq + 1 > batch_max_tokens:
        # the reference's np.pad would receive a negative pad width here
        raise ValueError(f"batch_max_tokens={batch_max_tokens} too small for {nseq} segments")
    total_lens = prefix_lens + causal_lens

    pad = batch_max_tokens - nseq
    cu = np.zeros(batch_max_tokens, dtype=np.int32)
    cu[1:nseq + 1] = np.cumsum(total_lens, dtype=np.int32)
    tensors = {
        "prefix_lens": np.concatenate([prefix_lens, np.zeros(pad, dtype=prefix_lens.dtype)]),
        "causal_lens": np.concatenate([causal_lens, np.zeros(pad, dtype=causal_lens.dtype)]),
        "cu_seqlens": cu,
    }
    scalars = {
        "total_seqlen": int(total_lens.sum()),
        "numseqs": nseq,
        "max_seqlen_prefix": int(prefix_lens.max()),
        "max_seqlen_causal": int(causal_lens.max()),
        "max_seqlen_all": int(total_lens.max()),
    }
    return tensors, scalars


def useful_entries(prefix_lens, causal_lens, is_causal: bool = False) -> int:
    """Number of attended (query, key) pairs per head.

    A query at local index i of a segment with prefix p attends key j iff
    j <= i or j < p (j <= i only when ``is_causal``). Summed over one segment of
    length L = p + c this is p*p + c*p + c*(c+1)/2 (or L*(L+1)/2).
    """
    p = np.asarray(prefix_lens, dtype=np.int64)
    c = np.asarray(causal_lens, dtype=np.int64)
    if is_causal:
        n = p + c
        return int((n * (n + 1) // 2).sum())
    return int((p * p + c * p + c * (c + 1) // 2).sum())


def useful_flops(prefix_lens, causal_lens, num_heads: int, head_dim: int,
                 is_causal: bool = False, fwd: bool = True, bwd: bool = True) -> int:
    """Useful FLOPs: 4*D per attended pair forward (QK^T, PV), 10*D backward
    (S recompute, dV, dP, dQ, dK), times heads."""
    n = useful_entries(prefix_lens, causal_lens, is_causal)
    per = (4 if fwd else 0) + (10 if bwd else 0)
    return per * head_dim * num_heads * n
