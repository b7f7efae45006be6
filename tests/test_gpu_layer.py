"""GPU: the fused attention layer (RoPE prologue, gated epilogue, their backward)
against the reference's unfused sequence (models/layers.py:131-155) built from
PyTorch ops around the same attention op, and the fused config-5 stack against
the float32 stack.

* RoPE forward: bitwise the fp32 PyTorch RoPE (same operation order).
* Gated output: bitwise sigmoid(gate) * attention except where a float32 sigmoid
  that differs in its last bits rounds to the neighbouring bf16 value.
* Gradients of the projection output: within the attention op's own bar (max-abs
  2e-2, mean-abs 2e-3) of autograd through the unfused sequence; the fused path
  rounds the gate and RoPE gradients once where autograd rounds twice.
"""
import numpy as np
import pytest
import torch

from oracle.prefixlm_oracle import attention_fwd
from prefixlm import flash_attn_varlen_prefixlm, fused_attention_layer
from prefixlm.hrm_stack import (FusedLayer, HRMStack, HRMStackConfig, apply_rotary, packed_position_ids,
                                rotary_cos_sin)
from prefixlm.layer import rope
from prefixlm.synth import metadata_tensors, segments_for_config

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _batch(prefix, causal, T, H, seed):
    st, ss = metadata_tensors(prefix, causal, T, DEV)
    pos = packed_position_ids(prefix, causal, T, DEV)
    cos, sin = rotary_cos_sin(pos, 128, 10000.0, 8192)
    g = torch.Generator(device="cpu").manual_seed(seed)
    gqkv = (torch.randn(T, 4 * H, 128, generator=g) * 1.5).to(DEV, torch.bfloat16)
    dy = torch.randn(T, H, 128, generator=g).to(DEV, torch.bfloat16)
    return {**st, **ss}, cos.contiguous(), sin.contiguous(), gqkv, dy


def _unfused(gqkv, cos, sin, is_causal, seq):
    H = gqkv.shape[1] // 4
    gate, q, k, v = gqkv.split((H, H, H, H), dim=1)
    q = apply_rotary(q, cos, sin)
    k = apply_rotary(k, cos, sin)
    o = flash_attn_varlen_prefixlm(q, k, v, is_causal, **seq)
    return torch.sigmoid(gate) * o


CASES = [([0, 130, 200], [300, 77, 0], 800, 2), ([5, 64, 128, 129], [123, 64, 1, 127], 700, 3)]


def _random_case(seed):
    """1-10 segments of 1-1200 rows (log-uniform), prefixes anywhere in [0, L], 0-150
    padding rows, 1-4 heads."""
    rng = np.random.default_rng(8800 + seed)
    n = int(rng.integers(1, 11))
    L = np.exp(rng.uniform(0, np.log(1200), size=n)).astype(np.int64) + 1
    p = np.floor(rng.uniform(size=n) * (L + 1)).astype(np.int64)
    return p.tolist(), (L - p).tolist(), int(L.sum()) + int(rng.integers(0, 151)), int(rng.integers(1, 5))


CASES += [_random_case(s) for s in range(6)]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_rope_kernel_matches_fp32_torch_rope(case):
    prefix, causal, T, H = CASES[case]
    print(f"[layer] rope case {case}", flush=True)
    seq, cos, sin, gqkv, _ = _batch(prefix, causal, T, H, 11 + case)
    x = gqkv[:, H:3 * H]
    y = torch.empty(T, 2 * H, 128, dtype=torch.bfloat16, device=DEV)
    rope(x, y, cos, sin)
    assert torch.equal(y, apply_rotary(x, cos, sin))
    # backward: the transpose of the rotation, against autograd of the fp32 RoPE
    dy = torch.randn(T, 2 * H, 128, device=DEV).to(torch.bfloat16)
    xf = x.float().requires_grad_()
    apply_rotary(xf, cos, sin).backward(dy.float())
    dx = dy.clone()
    rope(dx, dx, cos, sin, backward=True)
    err = (dx.float() - xf.grad).abs()
    assert err.max().item() <= 2 ** -8 * xf.grad.abs().max().item() + 1e-6


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("is_causal", [False, True])
def test_fused_layer_matches_unfused_sequence(case, is_causal):
    prefix, causal, T, H = CASES[case]
    print(f"[layer] case {case} is_causal={is_causal}", flush=True)
    seq, cos, sin, gqkv, dy = _batch(prefix, causal, T, H, 21 + case)
    g1 = gqkv.clone().requires_grad_()
    y1 = fused_attention_layer(g1, cos, sin, is_causal, **seq)
    y1.backward(dy)
    g2 = gqkv.clone().requires_grad_()
    y2 = _unfused(g2, cos, sin, is_causal, seq)
    y2.backward(dy)
    torch.cuda.synchronize()
    total = int(seq["total_seqlen"])
    diff = (y1.float() - y2.float()).abs()
    frac = (diff > 0).float().mean().item()
    print(f"[layer] y: max_abs={diff.max().item():.3e} differing={frac:.2e}", flush=True)
    assert diff.max().item() <= 1e-2 and frac <= 1e-3
    assert (y1[total:] == 0).all()
    for name, sl in (("dgate", slice(0, H)), ("dq", slice(H, 2 * H)), ("dk", slice(2 * H, 3 * H)),
                     ("dv", slice(3 * H, 4 * H))):
        a, b = g1.grad[:, sl].float(), g2.grad[:, sl].float()
        err = (a[:total] - b[:total]).abs()
        print(f"[layer] {name}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e} "
              f"max|ref|={b.abs().max().item():.3f}", flush=True)
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, name
        assert (a[total:] == 0).all(), name


def test_config5_fused_stack_within_its_own_floor():
    prefix, causal = segments_for_config(5)
    T = 16384
    st, ss = metadata_tensors(prefix, causal, T, DEV)
    seq = {**st, **ss}
    pos = packed_position_ids(prefix, causal, T, DEV)
    segs, cs = [], 0
    for p, c in zip(prefix, causal):
        segs.append((cs, int(p), int(p + c)))
        cs += int(p + c)
    base = HRMStack(HRMStackConfig(layers_per_module=1)).init_weights(1005)
    g = torch.Generator(device="cpu").manual_seed(1005)
    x = torch.randn(T, 2048, generator=g).to(torch.bfloat16).to(DEV)

    def ref_attn(q, k, v, is_causal, **_):
        return attention_fwd(q, k, v, segs, is_causal)[0].to(q.dtype)

    def model(dtype):
        m = HRMStack(HRMStackConfig(layers_per_module=1)).to(DEV)
        with torch.no_grad():
            for (_, p), (_, p0) in zip(m.named_parameters(), base.named_parameters()):
                p.copy_(p0.to(torch.bfloat16).float())
        return m.to(dtype)

    m16, ref = model(torch.bfloat16), model(torch.float32)
    with torch.no_grad():
        out_fused = m16(x, pos, FusedLayer(fused_attention_layer), seq)
        out_unfused = m16(x, pos, flash_attn_varlen_prefixlm, seq)
        out_ref = ref(x.float(), pos, ref_attn, seq)
    torch.cuda.synchronize()
    e_f = (out_fused.float() - out_ref).abs().max().item()
    e_u = (out_unfused.float() - out_ref).abs().max().item()
    print(f"[parity] cfg5 bf16 stack vs fp32 stack: fused layer {e_f:.3e}, unfused {e_u:.3e}", flush=True)
    assert torch.isfinite(out_fused).all()
    assert e_f <= max(3e-2, 1.5 * e_u)
