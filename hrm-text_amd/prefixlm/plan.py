"""Host-built work-list plans for a packed batch.

Every ``flash_attn_varlen_prefixlm`` call otherwise starts with a small device
kernel that turns the segment metadata into cost-ordered tile lists. A training
step makes many calls on the same batch (each layer and H/L cycle of the HRM
stack, forward and backward), so the lists can be built once on the host, where
the data loader already holds the metadata as numpy arrays
(dataset_new.py:129-134 calls ``compute_aux_seq_tensors_scalars`` there), and
travel with the batch::

    tensors, scalars = compute_aux_seq_tensors_scalars(seqlen_i, seqlen_o, T)
    tensors.update(plan_inputs(tensors, scalars, device))

``seq_info`` then carries ``plan`` (int32, on the device) and ``plan_ds_blocks``
(a 0-d int64 CPU tensor, like the reference's other scalars) to the op with the
other metadata; the op accepts both as optional keywords. ``plan_ds_blocks`` is the
number of stored-dS blocks per head the batch attends, which the backward's dS
buffer is sized to (without it the bound from ``max_seqlen_all`` is used).

The plan is a deterministic function of the metadata (the C builder sorts by
decreasing tile cost, ties by segment and tile), is valid for either ``is_causal``
(which only orders the lists; the dS layout follows ``prefix_lens`` either way), and
is rejected by the op when its size does not fit the call's ``total_seqlen`` and
``numseqs``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _capi

__all__ = ["build_plan", "plan_size", "plan_ds_blocks", "plan_inputs"]


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


def plan_ds_blocks(plan: np.ndarray) -> int:
    """Stored-dS blocks per head of the batch the host plan was built for."""
    a = np.ascontiguousarray(plan, dtype=np.int32)
    n = int(_capi.load().prefixlm_plan_ds_blocks(a.ctypes.data_as(ctypes.c_void_p), a.nbytes))
    if n < 0:
        raise ValueError("not a prefixlm plan")
    return n


def plan_inputs(tensors: dict, scalars: dict, device, is_causal: bool = False) -> dict:
    """``{"plan": int32 tensor on device, "plan_ds_blocks": 0-d int64 CPU tensor}`` for
    ``seq_info`` (the two optional keywords of the op)."""
    import torch
    p = build_plan(tensors, scalars, is_causal)
    return {"plan": torch.from_numpy(p).to(device),
            "plan_ds_blocks": torch.tensor(plan_ds_blocks(p), dtype=torch.int64)}
