"""Config 5: the HRM stack (hidden 2048, 16 x d128, SwiGLU 5632, RMSNorm, RoPE,
2 H x 2 L cycles, one layer per module, and 8 for the depth the benchmark runs) on
16384 packed tokens with config-2
segmentation, with the HIP attention, against the same stack in float32 with the
fp32 oracle attention.

* Parity bar (max-abs 3e-2 on the final output): the stack runs in float32 and only
  the attention call is bf16 (q, k, v rounded to bf16 in, bf16 out), so the
  difference measures the op inside the recurrence.
* All-bf16 stack: its own bf16 GEMMs and residual adds already move the output by
  ~8e-2 from float32 even with an exact attention; the test checks that the HIP op
  adds no more than that floor does.
"""
import pytest
import torch

from oracle.prefixlm_oracle import attention_fwd
from prefixlm import flash_attn_varlen_prefixlm
from prefixlm.hrm_stack import HRMStack, HRMStackConfig, packed_position_ids
from prefixlm.synth import metadata_tensors, segments_for_config

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _setup(layers=1):
    prefix, causal = segments_for_config(5)
    T = 16384
    st, ss = metadata_tensors(prefix, causal, T, DEV)
    pos = packed_position_ids(prefix, causal, T, DEV)
    segs, cs = [], 0
    for p, c in zip(prefix, causal):
        segs.append((cs, int(p), int(p + c)))
        cs += int(p + c)
    base = HRMStack(HRMStackConfig(layers_per_module=layers)).init_weights(1005)
    g = torch.Generator(device="cpu").manual_seed(1005)
    x = torch.randn(T, 2048, generator=g).to(torch.bfloat16).to(DEV)

    def ref_attn(q, k, v, is_causal, **_):
        return attention_fwd(q, k, v, segs, is_causal)[0].to(q.dtype)
    return {**st, **ss}, pos, base, x, ref_attn


def _model(base, attn_dtype, dtype):
    m = HRMStack(HRMStackConfig(layers_per_module=base.cfg.layers_per_module, attn_dtype=attn_dtype)).to(DEV)
    with torch.no_grad():
        for (_, p), (_, p0) in zip(m.named_parameters(), base.named_parameters()):
            p.copy_(p0.to(torch.bfloat16).float())       # bf16-representable weights everywhere
        m.zL_init.copy_(base.zL_init)
    return m.to(dtype)


def _report(tag, a, b):
    err = (a.float() - b.float()).abs()
    print(f"[parity] cfg5 {tag}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e} "
          f"max|ref|={b.abs().max().item():.3f}", flush=True)
    return err.max().item()


def test_config5_stack_attention_in_bf16():
    seq, pos, base, x, ref_attn = _setup()
    ours = _model(base, torch.bfloat16, torch.float32)
    ref = _model(base, None, torch.float32)
    with torch.no_grad():
        out = ours(x.float(), pos, flash_attn_varlen_prefixlm, seq)
        out_ref = ref(x.float(), pos, ref_attn, seq)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert _report("fp32 stack, HIP bf16 attention vs fp32 stack", out, out_ref) <= 3e-2


def test_config5_stack_8_layers_per_module_attention_in_bf16():
    """The depth the stack benchmark runs: 8 layers per module, 48 attention calls per
    forward, the same isolation of the op (float32 stack, bf16 attention call)."""
    seq, pos, base, x, ref_attn = _setup(layers=8)
    ours = _model(base, torch.bfloat16, torch.float32)
    ref = _model(base, None, torch.float32)
    with torch.no_grad():
        out = ours(x.float(), pos, flash_attn_varlen_prefixlm, seq)
        del ours
        out_ref = ref(x.float(), pos, ref_attn, seq)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert _report("8 layers/module: fp32 stack, HIP bf16 attention vs fp32 stack", out, out_ref) <= 3e-2


def test_config5_all_bf16_stack_within_its_own_floor():
    seq, pos, base, x, ref_attn = _setup()
    m16 = _model(base, None, torch.bfloat16)
    ref = _model(base, None, torch.float32)
    with torch.no_grad():
        out = m16(x, pos, flash_attn_varlen_prefixlm, seq)
        out_exact_attn = m16(x, pos, ref_attn, seq)
        out_ref = ref(x.float(), pos, ref_attn, seq)
    torch.cuda.synchronize()
    ours = _report("bf16 stack, HIP attention vs fp32 stack", out, out_ref)
    floor = _report("bf16 stack, fp32 attention vs fp32 stack", out_exact_attn, out_ref)
    assert torch.isfinite(out).all()
    assert ours <= max(3e-2, 1.5 * floor)


def test_config5_bf16_stack_fused_elementwise_and_layer():
    """The all-bf16 stack with the HIP SwiGLU / RMSNorm kernels and the fused attention
    layer: forward output and the gradient of the input, each within the floor the
    all-bf16 stack with PyTorch's elementwise ops and the unfused op already shows."""
    from prefixlm import fused_attention_layer
    from prefixlm.hrm_stack import FusedLayer
    seq, pos, base, x, ref_attn = _setup()
    m16 = _model(base, None, torch.bfloat16)
    ref = _model(base, None, torch.float32)
    dout = torch.randn(x.shape, generator=torch.Generator(device="cpu").manual_seed(7)).to(DEV)

    def run(model, xin, attn):
        xin = xin.detach().requires_grad_()
        # every module call with gradients, so that the input's gradient crosses all six
        out = model(xin, pos, attn, seq, bp_steps=None)
        (gx,) = torch.autograd.grad(out, xin, dout.to(out.dtype))
        return out.detach(), gx
    out_ref, gx_ref = run(ref, x.float(), ref_attn)
    out_plain, gx_plain = run(m16, x, flash_attn_varlen_prefixlm)
    m16.cfg.fused_elementwise = True
    out, gx = run(m16, x, FusedLayer(fused_attention_layer))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(gx).all()
    o_ours = _report("bf16 stack, fused elementwise + fused layer vs fp32 stack (out)", out, out_ref)
    o_plain = _report("bf16 stack, PyTorch elementwise + op vs fp32 stack (out)", out_plain, out_ref)
    g_ours = _report("bf16 stack, fused elementwise + fused layer vs fp32 stack (dx)", gx, gx_ref)
    g_plain = _report("bf16 stack, PyTorch elementwise + op vs fp32 stack (dx)", gx_plain, gx_ref)
    assert o_ours <= max(3e-2, 1.5 * o_plain)
    assert g_ours <= 1.5 * g_plain + 1e-3 * gx_ref.abs().max().item()
