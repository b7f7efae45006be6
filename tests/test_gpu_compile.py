"""The ops inside a compiled graph, as the reference compiles its train step
(`torch.compile(dynamic=False)`, pretrain.py:206): the varlen op, the fused attention
layer and the SwiGLU / RMSNorm ops traced with AOT autograd (fake kernels,
functionalization, the backward custom ops in the backward graph), forward values and
gradients bitwise equal to eager execution. The loss is linear in the outputs, so both
paths hand the backward the same output gradient."""
import pytest
import torch

from prefixlm import flash_attn_varlen_prefixlm, fused_attention_layer, rms_norm, swiglu
from prefixlm.hrm_stack import rotary_cos_sin
from prefixlm.synth import make_batch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _grads(fn, inputs, w):
    xs = [x.detach().clone().requires_grad_() for x in inputs]
    out = fn(*xs)
    loss = (out.float() * w).sum()
    gs = torch.autograd.grad(loss, xs)
    return out.detach(), gs


def _same(tag, a, b):
    print(f"[compile] {tag}: equal={torch.equal(a, b)}", flush=True)
    assert torch.equal(a, b), tag


def test_varlen_op_compiled_fwd_bwd_bitwise():
    b = make_batch([40, 200, 9], [90, 0, 150], 512, 4, 128, seed=11, device=DEV)
    seq = b.seq_info

    def f(q, k, v):
        return flash_attn_varlen_prefixlm(q, k, v, False, **seq)

    w = torch.randn(b.q.shape, generator=torch.Generator(device="cpu").manual_seed(3)).to(DEV)
    cf = torch.compile(f, backend="aot_eager", dynamic=False, fullgraph=True)
    out_e, g_e = _grads(f, (b.q, b.k, b.v), w)
    out_c, g_c = _grads(cf, (b.q, b.k, b.v), w)
    _same("varlen out", out_c, out_e)
    for name, a, e in zip("qkv", g_c, g_e):
        _same(f"varlen d{name}", a, e)


def test_layer_and_elementwise_compiled_fwd_bwd_bitwise():
    T, H, D, hid = 384, 4, 128, 512
    b = make_batch([100, 30], [60, 194], T, H, D, seed=12, device=DEV, with_dout=False)
    seq = b.seq_info
    pos = torch.cat([torch.arange(160), torch.arange(224)]).to(DEV)
    cos, sin = rotary_cos_sin(pos, D, 10000.0, 1024)
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(T, hid, generator=g).to(DEV, torch.bfloat16)
    w_gqkv = (torch.randn(4 * H * D, hid, generator=g) * 0.05).to(DEV, torch.bfloat16)
    w_gu = (torch.randn(2 * 256, H * D, generator=g) * 0.05).to(DEV, torch.bfloat16)

    def f(x, w_gqkv, w_gu):
        h = rms_norm(x, 1e-6)
        gqkv = torch.nn.functional.linear(h, w_gqkv).view(T, 4 * H, D)
        a = fused_attention_layer(gqkv, cos, sin, False, **seq).reshape(T, H * D)
        return swiglu(torch.nn.functional.linear(a, w_gu))

    w = torch.randn(T, 256, generator=g).to(DEV)
    cf = torch.compile(f, backend="aot_eager", dynamic=False, fullgraph=True)
    out_e, g_e = _grads(f, (x, w_gqkv, w_gu), w)
    out_c, g_c = _grads(cf, (x, w_gqkv, w_gu), w)
    _same("layer out", out_c, out_e)
    for name, a, e in zip(("x", "w_gqkv", "w_gu"), g_c, g_e):
        _same(f"layer d{name}", a, e)
