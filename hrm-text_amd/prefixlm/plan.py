"""Host-built work-list plans for a packed batch.

Every ``flash_attn_varlen_prefixlm`` call otherwise starts with a small device
kernel that turns the segment metadata into cost-ordered tile lists. A training
step makes many calls on the same batch (each layer and H/L cycle of the HRM
stack, forward and backward), so the lists can be built once on the host, where
the data loader already holds the metadata as numpy arrays
(dataset_new.py:129-134 calls ``compute_aux_seq_tensors_scalars`` there), and
travel with the batch::

    tensors, scalars = compute_aux_seq_tensors_scalars(seqlen_i, seqlen_o, T)
    tensors["plan"] = build_plan(tensors, scalars)

``seq_info`` then carries ``plan`` to the op with the other metadata; the op
accepts it as an optional keyword. The plan is a deterministic function of the
metadata (the C builder sorts by decreasing tile cost, ties by segment and
tile), is valid for either ``is_causal`` (which only orders the lists), and is
rejected by the op when its size does not fit the call's ``total_seqlen`` and
``numseqs``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _capi

__all__ = ["build_plan", "plan_size"]


def plan_size(total_seqlen: int, numseqs: int) -> int:
    """Bytes of the plan for a batch with these scalars."""
    return int(_capi.load().prefixlm_plan_size(int(total_seqlen), int(numseqs)))


def _host_i32(x, n: int, name: str) -> np.ndarray:
    if hasattr(x, "detach"):           # a torch tensor (CPU or device)
        x = x.detach().cpu().numpy()
    a = np.ascontiguousarray(np.asarray(x)[:n], dtype=np.int32)
    if a.shape[0] < n:
        raise ValueError(f"{name} holds {a.shape[0]} entries, {n} needed")
    return a


def build_plan(tensors: dict, scalars: dict, is_causal: bool = False) -> np.ndarray:
    """int32 array holding the plan for the batch described by the two dicts that
    ``compute_aux_seq_tensors_scalars`` returns (numpy arrays or tensors; ints or
    0-d tensors). Raises ``RuntimeError`` on inconsistent metadata."""
    lib = _capi.load()
    nseq = int(scalars["numseqs"])
    total = int(scalars["total_seqlen"])
    pre = _host_i32(tensors["prefix_lens"], nseq, "prefix_lens")
    cau = _host_i32(tensors["causal_lens"], nseq, "causal_lens")
    cu = _host_i32(tensors["cu_seqlens"], nseq + 1, "cu_seqlens")
    T = int(np.asarray(tensors["cu_seqlens"].shape[0]))
    nbytes = plan_size(total, nseq)
    out = np.zeros(nbytes // 4, dtype=np.int32)
    p32 = ctypes.POINTER(ctypes.c_int32)
    _capi.check(lib.prefixlm_plan_build(pre.ctypes.data_as(p32), cau.ctypes.data_as(p32),
                                        cu.ctypes.data_as(p32), nseq, total, T, 1 if is_causal else 0,
                                        out.ctypes.data_as(ctypes.c_void_p), nbytes),
                "prefixlm_plan_build")
    return out
