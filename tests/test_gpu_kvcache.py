"""GPU: KV-cache attention (flash_attn_with_kvcache) against the fp32 oracle, the
cache update, consistency of prefill + decode with the training op, and tracing
under torch.compile(fullgraph=True) as the reference's engine compiles it
(simple_inference_engine.py:105-112).

Tolerances as for the training op: max-abs 2e-2, mean-abs 2e-3 against the fp32
oracle on the same bf16 inputs; cache rows bitwise.
"""
import numpy as np
import pytest
import torch

from oracle.kvcache_oracle import kvcache_attention
from prefixlm import flash_attn_varlen_prefixlm, flash_attn_with_kvcache
from prefixlm.synth import metadata_tensors

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(B, S, H, Smax, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    return mk(B, S, H, 128), mk(B, S, H, 128), mk(B, S, H, 128), mk(B, Smax, H, 128), mk(B, Smax, H, 128)


def _cmp(tag, got, ref):
    err = (got.float().cpu() - ref).abs()
    print(f"[kvcache] {tag}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, tag


def _run(q, k, v, kc, vc, lens, causal):
    qd, kd, vd, kcd, vcd = (t.to(DEV) for t in (q, k, v, kc, vc))
    ld = lens.to(DEV) if isinstance(lens, torch.Tensor) else lens
    out = flash_attn_with_kvcache(qd, kcd, vcd, k=kd, v=vd, cache_seqlens=ld, causal=causal, num_splits=1)
    torch.cuda.synchronize()
    return out, kcd.cpu(), vcd.cpu()


@pytest.mark.parametrize("S", [1, 3])
@pytest.mark.parametrize("causal", [False, True])
def test_decode_matches_oracle(S, causal):
    B, H, Smax = 5, 4, 1100          # three 512-key splits, the last one partial
    print(f"[kvcache] decode S={S} causal={causal}", flush=True)
    q, k, v, kc, vc = _inputs(B, S, H, Smax, 10 + S)
    lens = torch.tensor([0, 1, 511, 900, Smax - S], dtype=torch.int32)
    out, kc2, vc2 = _run(q, k, v, kc, vc, lens, causal)
    ref, kref, vref = kvcache_attention(q, kc, vc, k, v, lens, causal)
    _cmp(f"decode S={S} causal={causal}", out, ref)
    assert torch.equal(kc2, kref) and torch.equal(vc2, vref)


@pytest.mark.parametrize("causal", [False, True])
def test_decode_without_new_rows_and_full_cache(causal):
    B, S, H, Smax = 3, 2, 2, 700
    q, _, _, kc, vc = _inputs(B, S, H, Smax, 20)
    lens = torch.tensor([2, 350, Smax], dtype=torch.int32)
    qd, kcd, vcd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    out = flash_attn_with_kvcache(qd, kcd, vcd, cache_seqlens=lens.to(DEV), causal=causal)
    ref, _, _ = kvcache_attention(q, kc, vc, None, None, lens, causal)
    _cmp(f"cache only causal={causal}", out, ref)
    assert torch.equal(kcd.cpu(), kc)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,S", [(1, 300), (2, 129)])
def test_prefill_matches_oracle(B, S, causal):
    H, Smax = 3, 512
    print(f"[kvcache] prefill B={B} S={S} causal={causal}", flush=True)
    q, k, v, kc, vc = _inputs(B, S, H, Smax, 30 + S)
    out, kc2, vc2 = _run(q, k, v, kc, vc, 0, causal)
    ref, kref, vref = kvcache_attention(q, kc, vc, k, v, 0, causal)
    _cmp(f"prefill B={B} S={S} causal={causal}", out, ref)
    assert torch.equal(kc2, kref) and torch.equal(vc2, vref)


def test_prefill_then_decode_matches_training_op():
    """The engine's loop: prefill a prompt of p tokens, then decode one token at a
    time; every output matches the training op's row for that token in a segment
    whose prefix is the prompt."""
    p, n_gen, H, Smax = 200, 24, 4, 512
    T = p + n_gen
    g = torch.Generator().manual_seed(40)
    q, k, v = (torch.randn(T, H, 128, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    st, ss = metadata_tensors(np.array([p]), np.array([n_gen]), T, DEV)
    train = flash_attn_varlen_prefixlm(q, k, v, False, **st, **ss)
    kc = torch.zeros(1, Smax, H, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    pre = flash_attn_with_kvcache(q[None, :p], kc, vc, k=k[None, :p], v=v[None, :p], cache_seqlens=0)
    err = [(pre[0] - train[:p]).abs().max().item()]
    lens = torch.tensor([p], dtype=torch.int32, device=DEV)
    for t in range(p, T):
        o = flash_attn_with_kvcache(q[None, t:t + 1], kc, vc, k=k[None, t:t + 1], v=v[None, t:t + 1],
                                    cache_seqlens=lens)
        err.append((o[0, 0] - train[t]).abs().max().item())
        lens.add_(1)
    torch.cuda.synchronize()
    print(f"[kvcache] engine loop vs training op: max_abs={max(err):.3e}", flush=True)
    assert max(err) <= 2e-2


def test_decode_traces_under_torch_compile():
    B, S, H, Smax = 2, 1, 2, 256
    q, k, v, kc, vc = (t.to(DEV) for t in _inputs(B, S, H, Smax, 50))
    lens = torch.tensor([10, 200], dtype=torch.int32, device=DEV)

    @torch.compile(dynamic=False, fullgraph=True)
    def step(q, k, v, kc, vc, lens):
        return flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=lens, num_splits=1)

    kc1, vc1 = kc.clone(), vc.clone()
    out = step(q, k, v, kc1, vc1, lens)
    kc2, vc2 = kc.clone(), vc.clone()
    ref = flash_attn_with_kvcache(q, kc2, vc2, k=k, v=v, cache_seqlens=lens)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
