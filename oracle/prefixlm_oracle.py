"""CPU/fp32 oracle for packed varlen PrefixLM attention -- TEST INFRASTRUCTURE.

Only the tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the CPU
baseline, as the thing timed on the host). The product path never calls it.

What it restates (reference = sapientinc/HRM-Text, read as text only):

* ``aux_seq_ref``: the metadata helper of
  models/flash_attention_prefixlm_v2.py:10-24, as plain Python loops.
* ``allowed_two_pass``: which key each query sees, written literally as the two
  FlashAttention-3 varlen passes of the reference forward
  (models/flash_attention_prefixlm_v2.py:110-128): pass 1 = prefix rows x prefix
  keys (``seqused_q = seqused_k = prefix_lens``, causal iff ``is_causal``);
  pass 2 = suffix rows (``cu_seqlens + prefix_lens``) x all keys of the segment,
  causal with FA's bottom-right alignment when seqlen_q != seqlen_k.
* ``mask_closed_form``: the same rule in closed form, ``j <= i or j < p``.
* ``attention_fwd``: fp32 softmax attention with that explicit mask, per
  segment; returns O and the natural-log LSE of the scaled scores, the
  quantities FA3 returns (reference :49-85, :131). Rows past ``total_seqlen``
  are zero (reference :130); their LSE is -inf.
* ``attention_fwd_sdpa``: the same forward through
  ``torch.nn.functional.scaled_dot_product_attention`` on the MATH backend with
  a boolean mask -- the CPU SDPA baseline.
* ``attention_bwd``: closed-form softmax-attention gradients in fp32 (the
  arithmetic of the reference backward, reference :152-212, without the
  two-pass split); padding rows get zero gradients (reference :209-211).
* ``attention_fwd_fp64`` / ``attention_bwd_fp64``: float64 numpy versions that
  evaluate the two-pass rule row by row, for tiny inputs and golden vectors.

How each function is pinned (tests/test_oracle.py): the metadata against the
hand-computed known answer; the mask forms against each other by brute force;
the forward against SDPA's own causal (p = 0) and unmasked (p = L) paths and
against the fp64 row loop; LSE against ``torch.logsumexp``; the backward
against autograd through ``attention_fwd`` and against float64 central finite
differences; everything against the committed golden vectors.
"""
from __future__ import annotations

import math

import numpy as np
import torch

__all__ = [
    "aux_seq_ref", "allowed_two_pass", "mask_closed_form", "segments_from_meta",
    "attention_fwd", "attention_fwd_sdpa", "attention_bwd",
    "attention_fwd_fp64", "attention_bwd_fp64",
]


# ---------------------------------------------------------------- metadata --
def aux_seq_ref(prefix_lens, causal_lens, batch_max_tokens):
    """Loop restatement of models/flash_attention_prefixlm_v2.py:10-24."""
    prefix_lens = [int(x) for x in prefix_lens]
    causal_lens = [int(x) for x in causal_lens]
    n = len(prefix_lens)
    pre = [0] * batch_max_tokens
    cau = [0] * batch_max_tokens
    cu = [0] * batch_max_tokens
    run = 0
    for s in range(n):
        pre[s] = prefix_lens[s]
        cau[s] = causal_lens[s]
        run += prefix_lens[s] + causal_lens[s]
        cu[s + 1] = run          # leading 0, then the running sums, then 0 padding
    totals = [a + b for a, b in zip(prefix_lens, causal_lens)]
    scalars = {
        "total_seqlen": sum(totals),
        "numseqs": n,
        "max_seqlen_prefix": max(prefix_lens),
        "max_seqlen_causal": max(causal_lens),
        "max_seqlen_all": max(totals),
    }
    return {"prefix_lens": pre, "causal_lens": cau, "cu_seqlens": cu}, scalars


def segments_from_meta(prefix_lens, causal_lens, cu_seqlens, numseqs):
    """[(start, prefix, length)] from reference-format metadata (any container)."""
    def as_list(x):
        if isinstance(x, torch.Tensor):
            return x.detach().cpu().tolist()
        return list(np.asarray(x).tolist())
    pre, cau, cu = as_list(prefix_lens), as_list(causal_lens), as_list(cu_seqlens)
    n = int(numseqs)
    return [(int(cu[s]), int(pre[s]), int(pre[s]) + int(cau[s])) for s in range(n)]


# -------------------------------------------------------------------- mask --
def allowed_two_pass(i, j, p, L, is_causal):
    """Does local query i see local key j in a segment of length L, prefix p?

    Literal reading of the two FA3 calls (reference :115-128):
      pass 1: q rows [0, p), k rows [0, p); causal (top-left = bottom-right,
              since seqlen_q == seqlen_k) iff is_causal.
      pass 2: q rows [p, L) (cu_seqlens_q = cu_seqlens + prefix_lens), k rows
              [0, L); causal with bottom-right alignment, so pass-row r sees
              keys <= r + (L - (L - p)).
    """
    if not (0 <= i < L and 0 <= j < L):
        return False
    if i < p:                               # pass 1
        if j >= p:
            return False
        return (j <= i) if is_causal else True
    r = i - p                               # pass 2
    c = L - p
    return j <= r + (L - c)


def mask_closed_form(p, L, is_causal, device="cpu"):
    """Bool [L, L] mask, True where query i sees key j: j <= i or j < p."""
    i = torch.arange(L, device=device).view(L, 1)
    j = torch.arange(L, device=device).view(1, L)
    m = j <= i
    if not is_causal:
        m = m | (j < p)
    return m


def _head_chunk(L, H, budget=1 << 27):
    return max(1, min(H, budget // max(1, L * L)))


# ------------------------------------------------------------- fp32 forward --
@torch.no_grad()
def attention_fwd(q, k, v, segments, is_causal=False, softmax_scale=None):
    """fp32 PrefixLM attention. q,k,v: [T,H,D] (any float dtype, upcast).

    Returns (out fp32 [T,H,D], lse fp32 [H,T]).
    """
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    dev = q.device
    out = torch.zeros((T, H, D), dtype=torch.float32, device=dev)
    lse = torch.full((H, T), float("-inf"), dtype=torch.float32, device=dev)
    for (cs, p, L) in segments:
        if L == 0:
            continue
        mask = mask_closed_form(p, L, is_causal, dev)
        hc = _head_chunk(L, H)
        for h0 in range(0, H, hc):
            h1 = min(H, h0 + hc)
            qs = q[cs:cs + L, h0:h1].float().transpose(0, 1).contiguous()     # [h, L, D]
            ks = k[cs:cs + L, h0:h1].float().transpose(0, 1).contiguous()
            vs = v[cs:cs + L, h0:h1].float().transpose(0, 1).contiguous()
            s = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
            s = s.masked_fill(~mask, float("-inf"))
            m = torch.logsumexp(s, dim=-1)                        # [h, L]
            pmat = torch.exp(s - m.unsqueeze(-1))
            o = torch.matmul(pmat, vs)                            # [h, L, D]
            out[cs:cs + L, h0:h1] = o.transpose(0, 1)
            lse[h0:h1, cs:cs + L] = m
    return out, lse


@torch.no_grad()
def attention_fwd_sdpa(q, k, v, segments, is_causal=False, softmax_scale=None):
    """Same forward through SDPA (MATH backend, boolean mask), fp32. Returns out."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.zeros((T, H, D), dtype=torch.float32, device=q.device)
    with sdpa_kernel(SDPBackend.MATH):
        for (cs, p, L) in segments:
            if L == 0:
                continue
            mask = mask_closed_form(p, L, is_causal, q.device)
            qs = q[cs:cs + L].float().transpose(0, 1).unsqueeze(0)
            ks = k[cs:cs + L].float().transpose(0, 1).unsqueeze(0)
            vs = v[cs:cs + L].float().transpose(0, 1).unsqueeze(0)
            o = torch.nn.functional.scaled_dot_product_attention(
                qs, ks, vs, attn_mask=mask, scale=scale)
            out[cs:cs + L] = o[0].transpose(0, 1)
    return out


# ------------------------------------------------------------ fp32 backward --
@torch.no_grad()
def attention_bwd(q, k, v, dout, segments, is_causal=False, softmax_scale=None):
    """Closed-form fp32 gradients (dq, dk, dv) [T,H,D] of PrefixLM attention.

    With P = softmax(scale*QK^T + mask): dV = P^T dO, dP = dO V^T,
    dS = P * (dP - rowsum(dP * P)), dQ = scale * dS K, dK = scale * dS^T Q.
    """
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    dev = q.device
    dq = torch.zeros((T, H, D), dtype=torch.float32, device=dev)
    dk = torch.zeros_like(dq)
    dv = torch.zeros_like(dq)
    for (cs, p, L) in segments:
        if L == 0:
            continue
        mask = mask_closed_form(p, L, is_causal, dev)
        hc = _head_chunk(L, H, budget=1 << 26)
        for h0 in range(0, H, hc):
            h1 = min(H, h0 + hc)
            sl = (slice(cs, cs + L), slice(h0, h1))
            qs, ks, vs, dos = (t[sl].float().transpose(0, 1).contiguous() for t in (q, k, v, dout))
            s = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
            s = s.masked_fill(~mask, float("-inf"))
            pm = torch.softmax(s, dim=-1)
            dv_ = torch.matmul(pm.transpose(1, 2).contiguous(), dos)
            dp = torch.matmul(dos, vs.transpose(1, 2).contiguous())
            delta = (dp * pm).sum(-1, keepdim=True)
            ds = pm * (dp - delta)
            dq_ = torch.matmul(ds, ks) * scale
            dk_ = torch.matmul(ds.transpose(1, 2).contiguous(), qs) * scale
            dq[sl] = dq_.transpose(0, 1)
            dk[sl] = dk_.transpose(0, 1)
            dv[sl] = dv_.transpose(0, 1)
    return dq, dk, dv


# ------------------------------------------------------------ fp64 row loop --
def attention_fwd_fp64(q, k, v, segments, is_causal=False, softmax_scale=None):
    """float64 numpy forward that asks ``allowed_two_pass`` for every pair.

    For tiny inputs only (O(T * L) Python calls). Returns (out, lse[H,T])."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = np.zeros((T, H, D))
    lse = np.full((H, T), -np.inf)
    for (cs, p, L) in segments:
        for i in range(L):
            keys = [j for j in range(L) if allowed_two_pass(i, j, p, L, is_causal)]
            kk = k[cs + np.array(keys)]                # [n, H, D]
            vv = v[cs + np.array(keys)]
            s = np.einsum("hd,nhd->hn", q[cs + i], kk) * scale
            mx = s.max(axis=1, keepdims=True)
            e = np.exp(s - mx)
            z = e.sum(axis=1, keepdims=True)
            out[cs + i] = np.einsum("hn,nhd->hd", e / z, vv)
            lse[:, cs + i] = (mx + np.log(z))[:, 0]
    return out, lse


def attention_bwd_fp64(q, k, v, dout, segments, is_causal=False, softmax_scale=None):
    """float64 numpy gradients, row by row from the two-pass rule (tiny inputs)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    T, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    dq = np.zeros_like(q)
    dk = np.zeros_like(q)
    dv = np.zeros_like(q)
    for (cs, p, L) in segments:
        for i in range(L):
            keys = cs + np.array([j for j in range(L) if allowed_two_pass(i, j, p, L, is_causal)])
            s = np.einsum("hd,nhd->hn", q[cs + i], k[keys]) * scale
            e = np.exp(s - s.max(axis=1, keepdims=True))
            pr = e / e.sum(axis=1, keepdims=True)                     # [H, n]
            dp = np.einsum("hd,nhd->hn", dout[cs + i], v[keys])       # [H, n]
            ds = pr * (dp - (pr * dp).sum(axis=1, keepdims=True))
            dq[cs + i] += scale * np.einsum("hn,nhd->hd", ds, k[keys])
            dk[keys] += scale * np.einsum("hn,hd->nhd", ds, q[cs + i])
            dv[keys] += np.einsum("hn,hd->nhd", pr, dout[cs + i])
    return dq, dk, dv
