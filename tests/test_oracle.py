"""Pins the fp32 oracle before it is trusted as the checker.

Each oracle function is tested against something it does not restate:
the literal two-pass reading of the reference (row loop), torch's own SDPA
paths for the special cases p = 0 (causal) and p = L (no mask), autograd of
SDPA, float64 finite differences, and the committed golden vectors. The last
test plants a mistake in the oracle and checks that these comparisons catch it.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.prefixlm_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _pack(prefix, causal, T, H, D, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn((T, H, D), generator=g, dtype=torch.float32).to(dtype) for _ in range(4))
    segs, cs = [], 0
    for p, c in zip(prefix, causal):
        segs.append((cs, p, p + c))
        cs += p + c
    assert cs <= T
    return q, k, v, do, segs


def test_mask_forms_agree():
    for L in range(0, 13):
        for p in range(0, L + 1):
            for causal in (False, True):
                m = orc.mask_closed_form(p, L, causal)
                for i in range(L):
                    for j in range(L):
                        assert bool(m[i, j]) == orc.allowed_two_pass(i, j, p, L, causal), (L, p, causal, i, j)


def test_mask_special_cases():
    L = 9
    assert torch.equal(orc.mask_closed_form(0, L, False), torch.ones(L, L, dtype=torch.bool).tril())
    assert orc.mask_closed_form(L, L, False).all()
    for p in range(L + 1):
        assert torch.equal(orc.mask_closed_form(p, L, True), torch.ones(L, L, dtype=torch.bool).tril())


CASES = [([3, 0, 5, 2], [4, 6, 0, 1], 24), ([0], [13], 16), ([7], [0], 8), ([1, 2], [1, 9], 15)]


@pytest.mark.parametrize("prefix,causal,T", CASES)
@pytest.mark.parametrize("is_causal", [False, True])
def test_forward_matches_fp64_row_loop(prefix, causal, T, is_causal):
    q, k, v, _, segs = _pack(prefix, causal, T, 3, 16, seed=1)
    out, lse = orc.attention_fwd(q, k, v, segs, is_causal)
    ref_o, ref_lse = orc.attention_fwd_fp64(q.numpy(), k.numpy(), v.numpy(), segs, is_causal)
    np.testing.assert_allclose(out.numpy(), ref_o, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), ref_lse, atol=2e-6, rtol=1e-5)
    total = segs[-1][0] + segs[-1][2]
    assert (out[total:] == 0).all() and torch.isinf(lse[:, total:]).all()


def test_forward_special_cases_match_sdpa():
    H, D = 4, 32
    q, k, v, _, segs = _pack([0, 21], [17, 0], 40, H, D, seed=2)
    out, lse = orc.attention_fwd(q, k, v, segs)
    # segment 0 (p = 0) is plain causal attention; segment 1 (p = L) is unmasked
    for (cs, p, L), causal in zip(segs, (True, False)):
        qs, ks, vs = (t[cs:cs + L].transpose(0, 1) for t in (q, k, v))
        ref = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal).transpose(0, 1)
        torch.testing.assert_close(out[cs:cs + L], ref, atol=1e-5, rtol=1e-5)
        if not causal:
            s = qs @ ks.transpose(1, 2) / math.sqrt(D)
            torch.testing.assert_close(lse[:, cs:cs + L], torch.logsumexp(s, -1), atol=1e-5, rtol=1e-5)


def test_lse_normalises_probabilities():
    q, k, v, _, segs = _pack([5, 3], [9, 4], 24, 2, 16, seed=3)
    _, lse = orc.attention_fwd(q, k, v, segs)
    for cs, p, L in segs:
        m = orc.mask_closed_form(p, L, False)
        s = torch.einsum("ihd,jhd->hij", q[cs:cs + L], k[cs:cs + L]) / 4.0
        pr = torch.exp(s - lse[:, cs:cs + L, None]) * m
        torch.testing.assert_close(pr.sum(-1), torch.ones(2, L), atol=1e-5, rtol=1e-5)


def test_sdpa_form_matches_explicit_form():
    q, k, v, _, segs = _pack([10, 0, 31], [22, 40, 5], 120, 4, 64, seed=4)
    for causal in (False, True):
        a, _ = orc.attention_fwd(q, k, v, segs, causal)
        b = orc.attention_fwd_sdpa(q, k, v, segs, causal)
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_matches_sdpa_autograd(is_causal):
    H, D = 3, 16
    q, k, v, do, segs = _pack([6, 0, 11], [9, 12, 0], 40, H, D, seed=5)
    dq, dk, dv = orc.attention_bwd(q, k, v, do, segs, is_causal)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    outs = []
    for cs, p, L in segs:
        m = orc.mask_closed_form(p, L, is_causal)
        o = F.scaled_dot_product_attention(*(t[cs:cs + L].transpose(0, 1) for t in (qg, kg, vg)),
                                           attn_mask=m)
        outs.append((o.transpose(0, 1) * do[cs:cs + L]).sum())
    torch.stack(outs).sum().backward()
    for got, ref in ((dq, qg.grad), (dk, kg.grad), (dv, vg.grad)):
        torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-4)


def test_backward_fp64_matches_finite_differences():
    prefix, causal = [2, 0], [3, 2]
    T, H, D = 8, 1, 4
    q, k, v, do, segs = _pack(prefix, causal, T, H, D, seed=6)
    q, k, v, do = (t.double().numpy() for t in (q, k, v, do))

    def loss(q_, k_, v_):
        o, _ = orc.attention_fwd_fp64(q_, k_, v_, segs)
        return float((o * do).sum())

    dq, dk, dv = orc.attention_bwd_fp64(q, k, v, do, segs)
    eps = 1e-6
    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            f1 = loss(*args)
            args[which][idx] -= 2 * eps
            f0 = loss(*args)
            num[idx] = (f1 - f0) / (2 * eps)
        np.testing.assert_allclose(grad, num, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("prefix,causal,T", CASES)
def test_backward_fp32_matches_fp64(prefix, causal, T):
    q, k, v, do, segs = _pack(prefix, causal, T, 2, 16, seed=7)
    got = orc.attention_bwd(q, k, v, do, segs)
    ref = orc.attention_bwd_fp64(q.numpy(), k.numpy(), v.numpy(), do.numpy(), segs)
    for g, r in zip(got, ref):
        np.testing.assert_allclose(g.numpy(), r, atol=1e-5, rtol=1e-4)
    total = segs[-1][0] + segs[-1][2]
    assert all((g[total:] == 0).all() for g in got)


def test_segment_permutation_permutes_outputs():
    prefix, causal = [4, 0, 9], [5, 7, 2]
    q, k, v, do, segs = _pack(prefix, causal, 27, 2, 16, seed=8)
    out, lse = orc.attention_fwd(q, k, v, segs)
    order = [2, 0, 1]
    rows = torch.cat([torch.arange(segs[s][0], segs[s][0] + segs[s][2]) for s in order])
    segs2, cs = [], 0
    for s in order:
        segs2.append((cs, segs[s][1], segs[s][2]))
        cs += segs[s][2]
    out2, lse2 = orc.attention_fwd(q[rows], k[rows], v[rows], segs2)
    torch.testing.assert_close(out2, out[rows], atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(lse2, lse[:, rows], atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("name", ["tiny_prefixlm", "tiny_causal", "d128_prefixlm"])
def test_oracle_matches_golden(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    pre, cau = z["prefix_lens"].tolist(), z["causal_lens"].tolist()
    segs, cs = [], 0
    for p, c in zip(pre, cau):
        segs.append((cs, p, p + c))
        cs += p + c
    q, k, v, do = (torch.from_numpy(z[n]) for n in ("q", "k", "v", "dout"))
    causal = bool(z["is_causal"])
    out, lse = orc.attention_fwd(q, k, v, segs, causal)
    dq, dk, dv = orc.attention_bwd(q, k, v, do, segs, causal)
    np.testing.assert_allclose(out.numpy(), z["out"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), z["lse"], atol=1e-5, rtol=1e-5)
    for g, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(g.numpy(), z[n], atol=1e-5, rtol=1e-4)


def test_planted_mask_mistake_is_caught(monkeypatch):
    """A strict j < i diagonal in the closed-form mask must fail the row-loop check."""
    q, k, v, _, segs = _pack([3, 0], [5, 6], 16, 2, 8, seed=9)
    good, _ = orc.attention_fwd(q, k, v, segs)
    ref, _ = orc.attention_fwd_fp64(q.numpy(), k.numpy(), v.numpy(), segs)
    np.testing.assert_allclose(good.numpy(), ref, atol=2e-6, rtol=1e-5)

    def bad_mask(p, L, is_causal, device="cpu"):
        i = torch.arange(L, device=device).view(L, 1)
        j = torch.arange(L, device=device).view(1, L)
        return (j < i) | (j < p) | ((i == 0) & (j == 0))
    monkeypatch.setattr(orc, "mask_closed_form", bad_mask)
    bad, _ = orc.attention_fwd(q, k, v, segs)
    assert np.abs(bad.numpy() - ref).max() > 1e-2


# ---------------------------------------------------------------- kv cache --
def _kv_inputs(B, S, H, D, Smax, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    return mk(B, S, H, D), mk(B, S, H, D), mk(B, S, H, D), mk(B, Smax, H, D), mk(B, Smax, H, D)


def test_kvcache_prefill_is_the_bidirectional_prefix_segment():
    from oracle.kvcache_oracle import kvcache_attention
    from oracle.prefixlm_oracle import attention_fwd
    q, k, v, kc, vc = _kv_inputs(1, 37, 2, 16, 64, 1)
    out, kc2, vc2 = kvcache_attention(q, kc, vc, k, v, 0, causal=False)
    ref, _ = attention_fwd(q[0], k[0], v[0], [(0, 37, 37)])
    assert torch.allclose(out[0], ref, atol=1e-5)
    assert torch.equal(kc2[0, :37], k[0]) and torch.equal(kc2[0, 37:], kc[0, 37:])
    # causal prefill is SDPA's causal path
    out_c, _, _ = kvcache_attention(q, kc, vc, k, v, 0, causal=True)
    sd = torch.nn.functional.scaled_dot_product_attention(
        q[0].float().transpose(0, 1), k[0].float().transpose(0, 1), v[0].float().transpose(0, 1),
        is_causal=True).transpose(0, 1)
    assert torch.allclose(out_c[0], sd, atol=1e-5)


def test_kvcache_decode_steps_are_rows_of_the_prefixlm_forward():
    """Prefill a prompt of p tokens, then decode g tokens one at a time (S = 1,
    not causal, as the reference's engine does): each output is the varlen op's row
    for that token in a segment whose prefix is the prompt."""
    from oracle.kvcache_oracle import kvcache_attention
    from oracle.prefixlm_oracle import attention_fwd
    p, g_tok, H, D, Smax = 11, 6, 2, 16, 32
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(p + g_tok, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    ref, _ = attention_fwd(q, k, v, [(0, p, p + g_tok)])
    kc = torch.zeros(1, Smax, H, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    out, kc, vc = kvcache_attention(q[None, :p], kc, vc, k[None, :p], v[None, :p], 0)
    assert torch.allclose(out[0], ref[:p], atol=1e-5)
    for t in range(p, p + g_tok):
        lens = torch.tensor([t], dtype=torch.int32)
        out, kc, vc = kvcache_attention(q[None, t:t + 1], kc, vc, k[None, t:t + 1], v[None, t:t + 1], lens)
        assert torch.allclose(out[0, 0], ref[t], atol=1e-5), t


@pytest.mark.parametrize("length,S", [(5, 3), (16, 7), (1, 2), (9, 1)])
def test_kvcache_with_cache_and_new_rows_is_the_tail_of_a_varlen_segment(length, S):
    """len cached rows plus S new rows: the causal call is the last S rows of the
    varlen oracle's causal segment (prefix 0) over all len + S tokens; the
    non-causal call is the last S rows of a fully bidirectional segment (prefix =
    len + S). The varlen oracle is pinned by the fp64 two-pass row loop above."""
    from oracle.kvcache_oracle import kvcache_attention
    from oracle.prefixlm_oracle import attention_fwd
    H, D, Smax = 2, 16, 40
    n = length + S
    g = torch.Generator().manual_seed(100 + length * 7 + S)
    q, k, v = (torch.randn(n, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    kc = torch.randn(1, Smax, H, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(1, Smax, H, D, generator=g).to(torch.bfloat16)
    kc[0, :length], vc[0, :length] = k[:length], v[:length]
    lens = torch.tensor([length], dtype=torch.int32)
    qn, kn, vn = q[None, length:], k[None, length:], v[None, length:]
    out_c, kc2, _ = kvcache_attention(qn, kc, vc, kn, vn, lens, causal=True)
    ref_c, _ = attention_fwd(q, k, v, [(0, 0, n)])
    assert torch.allclose(out_c[0], ref_c[length:], atol=1e-5)
    assert torch.equal(kc2[0, :n], k)
    out_b, _, _ = kvcache_attention(qn, kc, vc, kn, vn, lens, causal=False)
    ref_b, _ = attention_fwd(q, k, v, [(0, n, n)])
    assert torch.allclose(out_b[0], ref_b[length:], atol=1e-5)
    # the same with the cache length given as an int
    out_i, _, _ = kvcache_attention(qn, kc, vc, kn, vn, length, causal=True)
    assert torch.equal(out_i, out_c)


def test_kvcache_planted_off_by_len_diagonal_is_caught(monkeypatch):
    """A causal diagonal that forgets the cache length (j > i) must fail the check
    against the varlen segment."""
    import oracle.kvcache_oracle as kvo
    from oracle.prefixlm_oracle import attention_fwd
    length, S, H, D, Smax = 6, 4, 2, 16, 16
    n = length + S
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(n, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    kc = torch.zeros(1, Smax, H, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[0, :length], vc[0, :length] = k[:length], v[:length]
    ref, _ = attention_fwd(q, k, v, [(0, 0, n)])

    def run():
        out, _, _ = kvo.kvcache_attention(q[None, length:], kc, vc, k[None, length:], v[None, length:],
                                          length, causal=True)
        return out[0]
    assert torch.allclose(run(), ref[length:], atol=1e-5)

    def forgets_len(S_, lk, lk_full):
        j = torch.arange(lk).view(1, 1, lk)
        i = torch.arange(S_).view(1, S_, 1)
        return j > i
    monkeypatch.setattr(kvo, "causal_masked", forgets_len)
    assert (run() - ref[length:]).abs().max() > 1e-2
