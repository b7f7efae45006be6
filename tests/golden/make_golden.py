"""Writes the golden vectors under tests/golden/ (run from the repository root).

The reference ships no test vectors for this path (it has no attention tests and
its arithmetic lives in the un-vendored FlashAttention-3 extension), so these
fixtures come from this build's float64 evaluator, which applies the reference's
two FA3 passes literally, row by row (oracle.prefixlm_oracle.allowed_two_pass and
attention_fwd_fp64 / attention_bwd_fp64). Inputs are bf16-representable float32
values so the same fixture also feeds the bf16 GPU kernels.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "hrm-text_amd"))

from oracle.prefixlm_oracle import attention_bwd_fp64, attention_fwd_fp64  # noqa: E402
from prefixlm.metadata import compute_aux_seq_tensors_scalars  # noqa: E402

CASES = {
    # name: (prefix_lens, causal_lens, T, H, D, is_causal, seed)
    "tiny_prefixlm": ([3, 0, 5, 2], [4, 6, 0, 1], 24, 2, 8, False, 11),
    "tiny_causal": ([3, 0, 5, 2], [4, 6, 0, 1], 24, 2, 8, True, 11),
    "d128_prefixlm": ([20, 0, 9], [20, 16, 0], 72, 2, 128, False, 12),
}


def bf16_round(x):
    """Round float32 to the nearest bf16 value (ties to even), kept as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def make(name, prefix, causal, T, H, D, is_causal, seed):
    rng = np.random.default_rng(seed)
    q, k, v, do = (bf16_round(rng.standard_normal((T, H, D)).astype(np.float32)) for _ in range(4))
    tens, scal = compute_aux_seq_tensors_scalars(np.array(prefix, np.int32), np.array(causal, np.int32), T)
    cu = tens["cu_seqlens"]
    segs = [(int(cu[s]), prefix[s], prefix[s] + causal[s]) for s in range(len(prefix))]
    out, lse = attention_fwd_fp64(q, k, v, segs, is_causal)
    dq, dk, dv = attention_bwd_fp64(q, k, v, do, segs, is_causal)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(
        path, q=q, k=k, v=v, dout=do, prefix_lens=np.array(prefix, np.int32),
        causal_lens=np.array(causal, np.int32), num_tokens=T, is_causal=is_causal,
        out=out.astype(np.float32), lse=lse.astype(np.float32), dq=dq.astype(np.float32),
        dk=dk.astype(np.float32), dv=dv.astype(np.float32))
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    for name, args in CASES.items():
        make(name, *args)
