"""The HRM block stack around the op: structure and a tiny CPU run with a float32
attention (no GPU)."""
import torch

from oracle.prefixlm_oracle import attention_fwd
from prefixlm.hrm_stack import (HRMStack, HRMStackConfig, apply_rotary, intermediate_size,
                                packed_position_ids, rotary_cos_sin)
from prefixlm.synth import metadata_tensors


def test_intermediate_size_matches_config5():
    # find_multiple(round(4 * 2048 * 2/3), 256) = 5632 (models/transformer.py:42-46)
    assert intermediate_size(2048, 4.0) == 5632
    assert HRMStackConfig().ffn == 5632 and HRMStackConfig().head_dim == 128


def test_rotary_is_a_rotation_and_identity_at_position_zero():
    pos = torch.tensor([0, 1, 5, 0])
    cos, sin = rotary_cos_sin(pos, 8, 10000.0, 16)
    x = torch.randn(4, 2, 8)
    y = apply_rotary(x, cos, sin)
    torch.testing.assert_close(y[0], x[0])
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1))


def test_positions_restart_per_segment():
    pos = packed_position_ids([2, 0], [1, 3], 8, "cpu")
    assert pos.tolist() == [0, 1, 2, 0, 1, 2, 0, 0]


def test_tiny_stack_runs_and_segments_are_independent():
    cfg = HRMStackConfig(hidden_size=64, num_heads=2, layers_per_module=1, max_seq_len=64)
    prefix, causal = [3, 0, 5], [4, 6, 2]
    T = 24
    model = HRMStack(cfg).init_weights(5)
    st, ss = metadata_tensors(prefix, causal, T, "cpu")
    segs, cs = [], 0
    for p, c in zip(prefix, causal):
        segs.append((cs, p, p + c))
        cs += p + c

    def attn(q, k, v, is_causal, **_):
        return attention_fwd(q, k, v, segs, is_causal)[0]

    x = torch.randn(T, 64)
    pos = packed_position_ids(prefix, causal, T, "cpu")
    y = model(x, pos, attn, {**st, **ss})
    assert y.shape == (T, 64) and torch.isfinite(y).all()
    # changing segment 2's inputs leaves segments 0 and 1 unchanged
    x2 = x.clone()
    x2[13:] += 1.0
    y2 = model(x2, pos, attn, {**st, **ss})
    torch.testing.assert_close(y2[:13], y[:13])


def test_grad_windows_follow_the_reference_split():
    """H_bp = min(H_cycles, bp_steps - 1), L_bp = bp_steps - H_bp; the last H_bp H
    calls and the last L_bp L calls run with gradients
    (models/baselines/hrm_nocarry_bp_warmup.py:75-89)."""
    m = HRMStack(HRMStackConfig(hidden_size=64, num_heads=2, H_cycles=2, L_cycles=3, max_seq_len=64))
    assert m.grad_windows(2) == ({5}, {1})
    assert m.grad_windows(3) == ({5}, {0, 1})
    assert m.grad_windows(5) == ({3, 4, 5}, {0, 1})
    assert m.grad_windows(None) == (set(range(6)), {0, 1})
    m2 = HRMStack(HRMStackConfig(hidden_size=64, num_heads=2, H_cycles=2, L_cycles=2, max_seq_len=64))
    assert m2.grad_windows(2) == ({3}, {1})


def test_only_the_window_records_gradients():
    cfg = HRMStackConfig(hidden_size=64, num_heads=2, layers_per_module=1, max_seq_len=64)
    prefix, causal = [3, 5], [4, 4]
    T = 16
    model = HRMStack(cfg).init_weights(5)
    assert model.zL_init.dtype == torch.bfloat16 and "zL_init" not in dict(model.named_parameters())
    st, ss = metadata_tensors(prefix, causal, T, "cpu")
    segs = [(0, 3, 7), (7, 5, 9)]
    seen = []

    def attn(q, k, v, is_causal, **_):
        seen.append(torch.is_grad_enabled())
        return attention_fwd(q, k, v, segs, is_causal)[0]

    x = torch.randn(T, 64, requires_grad=True)
    pos = packed_position_ids(prefix, causal, T, "cpu")
    y = model(x, pos, attn, {**st, **ss})          # reference default: bp_steps = 2
    # call order L0 L1 H0 L2 L3 H1: only L3 and H1 run with gradients
    assert seen == [False, False, False, False, True, True]
    y.sum().backward()
    assert x.grad is None                         # x reaches the window only through no-grad calls
    seen.clear()
    y_all = model(x, pos, attn, {**st, **ss}, bp_steps=None)
    assert seen == [True] * 6
    torch.testing.assert_close(y_all, y)
