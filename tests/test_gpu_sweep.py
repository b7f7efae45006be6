"""GPU: a sweep of seeded random packings against the fp32 oracle, at the bars of
tests/test_gpu_parity.py (O, dQ, dK, dV max-abs 2e-2 and mean-abs 2e-3; LSE 1e-3;
padding rows exactly zero).

The cases mix three families: many short segments (up to 400 rows), a few medium ones
(up to 1500) and a few long ones (up to 5000), prefixes anywhere in [0, L] with extra
weight on 0 and L, 1-8 heads, head dim 128 or (one in four) 64, either is_causal.

One exception to the absolute bar is stated here because no bf16 output can avoid it:
where |ref| >= 8 the bf16 grid spacing is 6.25e-2, so an element whose fp32 value sits
near the middle between two bf16 neighbours is 3.1e-2 from both. An element above 2e-2
passes only if the kernel's bf16 value is within one bf16 ulp of bf16(ref) there (a
5000-case run of this sweep met one such element: dV = 8.086, returned exactly as
bf16(ref) = 8.0625)."""
import numpy as np
import pytest
import torch

from oracle.prefixlm_oracle import attention_bwd, attention_fwd
from prefixlm import flash_attn_varlen_prefixlm, op
from prefixlm.synth import make_batch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
MAX_ABS, MEAN_ABS, LSE_ABS = 2e-2, 2e-3, 1e-3
N_CASES = 300


def _case(c):
    rng = np.random.default_rng(40000 + c)
    kind = c % 3
    n = int(rng.integers(1, 30 if kind == 0 else 6))
    hi = (400, 1500, 5000)[kind]
    L = np.exp(rng.uniform(0, np.log(hi), size=n)).astype(np.int64) + 1
    u = rng.uniform(size=n)
    p = np.where(u < 0.1, 0, np.where(u > 0.9, L, np.floor(rng.uniform(size=n) * (L + 1)))).astype(np.int64)
    p = np.minimum(p, L)
    T = int(L.sum()) + int(rng.integers(0, 200))
    H = int(rng.integers(1, 9))
    D = 64 if rng.uniform() < 0.25 else 128
    is_causal = bool(rng.integers(0, 2))
    return p, L, T, H, D, is_causal


def _check(name, got, ref, total, tag):
    g = got.float()[:total]
    r = ref[:total]
    err = (g - r).abs()
    mx = err.max().item() if err.numel() else 0.0
    mean = err.mean().item() if err.numel() else 0.0
    assert mean <= MEAN_ABS, f"{tag} {name}: mean {mean:.3e}"
    if mx > MAX_ABS:
        sel = err > MAX_ABS
        rb = r[sel].to(torch.bfloat16).float()
        ulp = torch.ldexp(torch.ones_like(rb), torch.frexp(rb).exponent - 8)
        k_ulps = ((g[sel] - rb).abs() / ulp).max().item()
        print(f"[sweep] {tag} {name}: max_abs={mx:.3e} above the bar where min|ref|="
              f"{r[sel].abs().min().item():.3f}, kernel within {k_ulps:.2f} bf16 ulp of bf16(ref)", flush=True)
        assert r[sel].abs().min().item() >= 8.0 and k_ulps <= 1.0, f"{tag} {name}: max {mx:.3e}"
    if total < got.shape[0]:
        assert (got[total:] == 0).all(), f"{tag} {name}: padding rows not zero"
    return mx


def test_random_packing_sweep():
    worst = {}
    for c in range(N_CASES):
        p, L, T, H, D, is_causal = _case(c)
        tag = f"sweep{c} n={len(L)} T={T} H={H} D={D} causal={is_causal}"
        b = make_batch(p, L - p, T, H, D, seed=40000 + c, device=DEV)
        segs, cs = [], 0
        for pp, ll in zip(p, L):
            segs.append((cs, int(pp), int(ll)))
            cs += int(ll)
        total = int(L.sum())
        q, k, v = (t.detach().clone().requires_grad_() for t in (b.q, b.k, b.v))
        out = flash_attn_varlen_prefixlm(q, k, v, is_causal, **b.seq_info)
        out.backward(b.dout)
        ref_o, ref_lse = attention_fwd(b.q, b.k, b.v, segs, is_causal, None)
        ref_g = attention_bwd(b.q, b.k, b.v, b.dout, segs, is_causal, None)
        for name, got, ref in zip(("out", "dq", "dk", "dv"), (out, q.grad, k.grad, v.grad), (ref_o, *ref_g)):
            mx = _check(name, got, ref, total, tag)
            worst[name] = max(worst.get(name, 0.0), mx)
        _, lse, _, _ = op.varlen_fwd(b.q, b.k, b.v, is_causal, *b.seq_info.values(), float(1.0 / np.sqrt(D)))
        lerr = (lse[:, :total] - ref_lse[:, :total]).abs().max().item()
        assert lerr <= LSE_ABS, f"{tag} lse {lerr:.3e}"
        worst["lse"] = max(worst.get("lse", 0.0), lerr)
    print("[sweep] " + ", ".join(f"{k} worst {v:.3e}" for k, v in worst.items()), flush=True)
