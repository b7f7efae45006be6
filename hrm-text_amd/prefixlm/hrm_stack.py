"""HRM recurrent block stack that calls the PrefixLM attention (the op's caller).

A from-scratch module stack with the reference's structure, used to check the op
end to end inside the H/L cycles (benchmark config 5):

* attention layer (models/layers.py:116-155): one fused gate/q/k/v projection
  split per head (:131-135), fp32 rotary embedding on q and k (:23-38, :138-140),
  the attention op (:145), ``sigmoid(gate) * attn`` and the output projection
  (:154-155);
* SwiGLU MLP with a fused gate/up projection (:158-168); intermediate size
  ``find_multiple(round(expansion * hidden * 2 / 3), 256)`` (models/transformer.py:42-46);
* pre-norm block ``x + attn(norm x); x + mlp(norm x)`` with ``F.rms_norm``
  (models/transformer.py:86-92) and a final norm (:114-116); with
  ``fused_elementwise`` the SwiGLU product and the norms run as HIP kernels
  (``prefixlm.swiglu``, ``prefixlm.rms_norm``);
* HRM recurrence (models/baselines/hrm_nocarry_bp_warmup.py:34-43, :75-91):
  separate H and L stacks, per H-cycle ``L_cycles`` L-calls on ``z_L + z_H`` then
  one H-call on ``z_H + z_L``, starting from ``z_H = x`` and ``zL_init``, a bf16
  buffer drawn from N(0, 1) (:65). Only the last ``bp_steps`` module calls run with
  gradients (H calls first, at least one L call; :75-89); the earlier calls run
  under ``torch.set_grad_enabled(False)``. The reference's default is 2.

The attention callable is injected, so the same weights run with the HIP op
(bf16) or with a float32 reference attention in tests. Wrapped in ``FusedLayer``
the callable instead receives the projection output [T, 4H, D] and cos/sin and
applies RoPE and the gate itself (``prefixlm.fused_attention_layer``). Weights
are drawn from N(0, std) with a seeded generator.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn.functional as F
from torch import Tensor, nn

__all__ = ["HRMStackConfig", "HRMStack", "FusedLayer", "rotary_cos_sin", "apply_rotary", "intermediate_size"]


def intermediate_size(hidden: int, expansion: float) -> int:
    n = round(expansion * hidden * 2 / 3)
    return -(n // -256) * 256


@dataclass
class HRMStackConfig:
    hidden_size: int = 2048
    num_heads: int = 16
    expansion: float = 4.0
    layers_per_module: int = 1
    H_cycles: int = 2
    L_cycles: int = 2
    norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    max_seq_len: int = 8192
    init_std: float = 0.02
    attn_causal: bool = False          # attn_type "causal" vs "prefixlm"
    # dtype q/k/v are cast to for the attention call (output cast back); None keeps
    # the stack's dtype. bfloat16 with a float32 stack isolates the op's precision.
    attn_dtype: Optional[torch.dtype] = None
    # SwiGLU and RMSNorm through the HIP kernels (prefixlm.swiglu / prefixlm.rms_norm,
    # bf16 only) instead of PyTorch's elementwise ops
    fused_elementwise: bool = False
    # in calls without gradients: the MLP's pre-norm and SwiGLU fused into the gate_up
    # projection (prefixlm.norm_mlp.rms_norm_swiglu, bf16; forward only, so calls with
    # gradients keep the separate ops). The attention's gqkv projection keeps the
    # library GEMM after the norm kernel: at 2048 -> 8192 columns that pair is faster
    # than the fused GEMM (rms_norm_linear stays available on its own).
    fused_gemm: bool = False

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def ffn(self) -> int:
        return intermediate_size(self.hidden_size, self.expansion)


def rotary_cos_sin(position_ids: Tensor, head_dim: int, theta: float, max_seq_len: int):
    """cos/sin [T, head_dim] in float32 for the given positions (half-split layout)."""
    dev = position_ids.device
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=dev) / head_dim))
    t = torch.arange(max_seq_len, dtype=torch.float32, device=dev)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[position_ids], emb.sin()[position_ids]


def apply_rotary(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """x [T, H, D]; rotation computed in float32 and cast back to x's dtype."""
    xf = x.float()
    half = x.shape[-1] // 2
    rot = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
    return (xf * cos.unsqueeze(-2) + rot * sin.unsqueeze(-2)).to(x.dtype)


AttnFn = Callable[..., Tensor]   # (q, k, v, is_causal, **seq_info) -> [T, H, D]


class FusedLayer:
    """An attention callable taking (gqkv [T, 4H, D], cos, sin, is_causal, **seq_info)
    and returning sigmoid(gate) * attention [T, H, D]: RoPE and the gate are its own."""

    def __init__(self, fn: Callable[..., Tensor]):
        self.fn = fn

    def __call__(self, *args, **kwargs) -> Tensor:
        return self.fn(*args, **kwargs)


class _Attention(nn.Module):
    def __init__(self, cfg: HRMStackConfig):
        super().__init__()
        self.cfg = cfg
        h, d = cfg.num_heads, cfg.head_dim
        self.gqkv = nn.Parameter(torch.empty(4 * h * d, cfg.hidden_size))
        self.o = nn.Parameter(torch.empty(cfg.hidden_size, h * d))

    def forward(self, x: Tensor, cos: Tensor, sin: Tensor, attn: AttnFn, seq_info: dict,
                prenormed: bool = True) -> Tensor:
        h, d = self.cfg.num_heads, self.cfg.head_dim
        if prenormed:
            g = F.linear(x, self.gqkv)
        else:
            # x still needs the block's pre-norm: it runs inside the projection GEMM
            from .norm_mlp import rms_norm_linear
            g = rms_norm_linear(x, self.gqkv, self.cfg.norm_eps)
        g = g.view(x.shape[0], 4 * h, d)
        if isinstance(attn, FusedLayer):
            o = attn(g, cos, sin, self.cfg.attn_causal, **seq_info)
            return F.linear(o.reshape(x.shape[0], h * d), self.o)
        gate, q, k, v = g.split((h, h, h, h), dim=1)   # v stays a strided view
        q = apply_rotary(q, cos, sin)
        k = apply_rotary(k, cos, sin)
        if self.cfg.attn_dtype is not None and self.cfg.attn_dtype != x.dtype:
            q, k, v = (t.to(self.cfg.attn_dtype) for t in (q, k, v))
        o = attn(q, k, v, self.cfg.attn_causal, **seq_info).to(x.dtype)
        return F.linear((torch.sigmoid(gate) * o).reshape(x.shape[0], h * d), self.o)


def _rms_norm(x: Tensor, cfg: HRMStackConfig) -> Tensor:
    if cfg.fused_elementwise:
        from .norm_mlp import rms_norm
        return rms_norm(x, cfg.norm_eps)
    return F.rms_norm(x, (x.shape[-1],), eps=cfg.norm_eps)


class _SwiGLU(nn.Module):
    def __init__(self, cfg: HRMStackConfig):
        super().__init__()
        self.cfg = cfg
        self.gate_up = nn.Parameter(torch.empty(2 * cfg.ffn, cfg.hidden_size))
        self.down = nn.Parameter(torch.empty(cfg.hidden_size, cfg.ffn))

    def forward(self, x: Tensor, prenormed: bool = True) -> Tensor:
        if not prenormed:
            # pre-norm, gate_up projection and SwiGLU in one GEMM
            from .norm_mlp import rms_norm_swiglu
            return F.linear(rms_norm_swiglu(x, self.gate_up, self.cfg.norm_eps), self.down)
        gu = F.linear(x, self.gate_up)
        if self.cfg.fused_elementwise:
            from .norm_mlp import swiglu
            return F.linear(swiglu(gu), self.down)
        gate, up = gu.chunk(2, dim=-1)
        return F.linear(F.silu(gate) * up, self.down)


class _Block(nn.Module):
    def __init__(self, cfg: HRMStackConfig):
        super().__init__()
        self.cfg = cfg
        self.attn = _Attention(cfg)
        self.mlp = _SwiGLU(cfg)

    def norm(self, x):
        return _rms_norm(x, self.cfg)

    def forward(self, x, cos, sin, attn, seq_info):
        x = x + self.attn(self.norm(x), cos, sin, attn, seq_info)
        if self.cfg.fused_gemm and not torch.is_grad_enabled():
            return x + self.mlp(x, prenormed=False)
        return x + self.mlp(self.norm(x))


class _Module(nn.Module):
    """One recurrent module (H or L): input injection, layers, final norm."""

    def __init__(self, cfg: HRMStackConfig):
        super().__init__()
        self.cfg = cfg
        self.layers = nn.ModuleList(_Block(cfg) for _ in range(cfg.layers_per_module))

    def forward(self, hidden, injection, cos, sin, attn, seq_info):
        x = hidden + injection
        for layer in self.layers:
            x = layer(x, cos, sin, attn, seq_info)
        return _rms_norm(x, self.cfg)


class HRMStack(nn.Module):
    """H and L modules run for H_cycles x L_cycles on one packed batch."""

    def __init__(self, cfg: HRMStackConfig):
        super().__init__()
        self.cfg = cfg
        self.H = _Module(cfg)
        self.L = _Module(cfg)
        # bf16 whatever the stack's dtype, as in the reference (a buffer, not trained)
        self.register_buffer("zL_init", torch.zeros(cfg.hidden_size, dtype=torch.bfloat16))

    @torch.no_grad()
    def init_weights(self, seed: int):
        g = torch.Generator(device="cpu").manual_seed(seed)
        for _, p in sorted(self.named_parameters()):
            p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float32) * self.cfg.init_std)
        self.zL_init.copy_(torch.randn(self.zL_init.shape, generator=g, dtype=torch.float32))
        return self

    def grad_windows(self, bp_steps: Optional[int]):
        """(L calls, H calls) that run with gradients: the last L_bp L calls and the
        last H_bp H calls, H_bp = min(H_cycles, bp_steps - 1), L_bp = bp_steps - H_bp
        (models/baselines/hrm_nocarry_bp_warmup.py:75-79); every call when bp_steps
        is None."""
        cfg = self.cfg
        n_l, n_h = cfg.H_cycles * cfg.L_cycles, cfg.H_cycles
        if bp_steps is None:
            return set(range(n_l)), set(range(n_h))
        h_bp = min(n_h, bp_steps - 1)
        l_bp = bp_steps - h_bp
        return {k for k in range(n_l) if k >= n_l - l_bp}, {i for i in range(n_h) if i >= n_h - h_bp}

    def forward(self, x: Tensor, position_ids: Tensor, attn: AttnFn, seq_info: dict,
                bp_steps: Optional[int] = 2) -> Tensor:
        cfg = self.cfg
        cos, sin = rotary_cos_sin(position_ids, cfg.head_dim, cfg.rope_theta, cfg.max_seq_len)
        l_grad, h_grad = self.grad_windows(bp_steps)
        grad_on = torch.is_grad_enabled()
        z_H = x
        z_L = self.zL_init.to(x.dtype).expand_as(x)
        for i in range(cfg.H_cycles):
            for k in range(i * cfg.L_cycles, (i + 1) * cfg.L_cycles):
                with torch.set_grad_enabled(grad_on and k in l_grad):
                    z_L = self.L(z_L, z_H, cos, sin, attn, seq_info)
            with torch.set_grad_enabled(grad_on and i in h_grad):
                z_H = self.H(z_H, z_L, cos, sin, attn, seq_info)
        return z_H


def packed_position_ids(prefix, causal, T: int, device) -> Tensor:
    """Positions restart at 0 for every segment; padding rows get 0
    (dataset_new.py:110-111, :119-127)."""
    pos = torch.zeros(T, dtype=torch.long)
    cs = 0
    for p, c in zip(prefix, causal):
        L = int(p) + int(c)
        pos[cs:cs + L] = torch.arange(L)
        cs += L
    return pos.to(device)
