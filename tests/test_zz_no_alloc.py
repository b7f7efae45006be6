"""GPU: prefixlm_bwd_noalloc (the backward with the library's own scratch, no workspace,
no allocation) against prefixlm_bwd with a caller workspace, through the C ABI: two calls
in a row, the second on a smaller batch, each bitwise equal (same kernels, same item
order), with device-built lists and with a host plan."""
import ctypes

import numpy as np
import pytest
import torch

from prefixlm import _capi, build_plan, op
from prefixlm.synth import make_batch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _bwd_args(b, out, lse, out_lo, q_amax, dq, dk, dv, ws, plan):
    T, H, D = b.q.shape
    st, sc = b.seq_tensors, b.seq_scalars
    P = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    return _capi.BwdArgs(
        q=P(b.q), k=P(b.k), v=P(b.v), out=P(out), out_lo=P(out_lo), dout=P(b.dout), lse=P(lse), q_amax=P(q_amax),
        dq=P(dq), dk=P(dk), dv=P(dv),
        q_stride_t=H * D, q_stride_h=D, k_stride_t=H * D, k_stride_h=D, v_stride_t=H * D, v_stride_h=D,
        out_stride_t=H * D, out_stride_h=D, out_lo_stride_t=H * D, out_lo_stride_h=D,
        dout_stride_t=H * D, dout_stride_h=D, dq_stride_t=H * D, dq_stride_h=D,
        dk_stride_t=H * D, dk_stride_h=D, dv_stride_t=H * D, dv_stride_h=D,
        prefix_lens=P(st["prefix_lens"]), causal_lens=P(st["causal_lens"]), cu_seqlens=P(st["cu_seqlens"]),
        meta_len=T, num_tokens=T, num_heads=H, head_dim=D,
        total_seqlen=int(sc["total_seqlen"]), numseqs=int(sc["numseqs"]),
        max_seqlen_prefix=int(sc["max_seqlen_prefix"]), max_seqlen_causal=int(sc["max_seqlen_causal"]),
        max_seqlen_all=int(sc["max_seqlen_all"]), is_causal=0, softmax_scale=float(1.0 / np.sqrt(D)),
        workspace=P(ws), workspace_bytes=ws.numel() if ws is not None else 0,
        plan=P(plan), plan_bytes=plan.numel() * 4 if plan is not None else 0)


def _both(b, use_plan):
    lib = _capi.load()
    T, H, D = b.q.shape
    sc = 1.0 / np.sqrt(D)
    out, lse, out_lo, q_amax = op.varlen_fwd(b.q, b.k, b.v, False, *b.seq_info.values(), sc)
    plan = torch.from_numpy(build_plan(b.seq_tensors, b.seq_scalars)).to(DEV) if use_plan else None
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = []
    for noalloc in (False, True):
        dq, dk, dv = (torch.full_like(b.q, float("nan")) for _ in range(3))
        ws = None
        if not noalloc:
            n = lib.prefixlm_bwd_workspace_size(T, H, D, int(b.seq_scalars["total_seqlen"]),
                                                int(b.seq_scalars["numseqs"]))
            ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        a = _bwd_args(b, out, lse, out_lo, q_amax, dq, dk, dv, ws, plan)
        fn = lib.prefixlm_bwd_noalloc if noalloc else lib.prefixlm_bwd
        rc = fn(ctypes.byref(a), stream)
        assert rc == 0, _capi.last_error()
        torch.cuda.synchronize()
        res.append((dq, dk, dv))
    return res


@pytest.mark.parametrize("use_plan", [False, True])
def test_noalloc_backward_matches_workspace_backward(use_plan):
    lib = _capi.load()
    assert lib.prefixlm_bwd_noalloc_max_scratch() == 16 << 20
    # first a larger batch (every segment kind, padding rows), then a smaller one: the
    # second call reuses the scratch the first left behind
    for prefix, causal, T, H, seed in (([0, 300, 77, 512], [700, 200, 900, 0], 3000, 8, 11),
                                       ([40, 0], [25, 70], 160, 3, 12)):
        print(f"[noalloc] plan={use_plan} T={T} H={H}", flush=True)
        b = make_batch(prefix, causal, T, H, 128, seed=seed, device=DEV)
        (rq, rk, rv), (gq, gk, gv) = _both(b, use_plan)
        for name, x, y in (("dq", rq, gq), ("dk", rk, gk), ("dv", rv, gv)):
            assert torch.isfinite(x).all(), name
            assert torch.equal(x, y), name


def test_noalloc_rejects_workspace_and_oversized_calls():
    lib = _capi.load()
    a = _capi.BwdArgs()
    a.workspace, a.workspace_bytes = 256, 256
    assert lib.prefixlm_bwd_noalloc(ctypes.byref(a), None) == 1 and "workspace" in _capi.last_error()
    a = _capi.BwdArgs()
    a.num_tokens, a.num_heads, a.head_dim, a.total_seqlen, a.numseqs = 1 << 20, 16, 128, 1 << 20, 1
    assert lib.prefixlm_bwd_noalloc(ctypes.byref(a), None) == 1 and "scratch" in _capi.last_error()
