"""GPU: calls given a host-built work-list plan produce bitwise the outputs of the
device-built lists (every work item is computed independently, so the item order
cannot change a result), and a plan sized for other metadata is rejected."""
import zlib

import numpy as np
import pytest
import torch

from prefixlm import build_plan, flash_attn_varlen_prefixlm, op
from prefixlm.synth import make_batch, make_config_batch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _fwd_bwd(b, is_causal, plan):
    q, k, v = (t.detach().clone().requires_grad_() for t in (b.q, b.k, b.v))
    out = flash_attn_varlen_prefixlm(q, k, v, is_causal, **b.seq_info, plan=plan)
    out.backward(b.dout)
    sc = 1.0 / np.sqrt(b.q.shape[-1])
    _, lse, lo, _ = op.varlen_fwd(b.q, b.k, b.v, is_causal, *b.seq_info.values(), sc, plan)
    torch.cuda.synchronize()
    return out.detach(), lse, lo, q.grad, k.grad, v.grad


def _plan_of(b, is_causal):
    return torch.from_numpy(build_plan(b.seq_tensors, b.seq_scalars, is_causal)).to(DEV)


CASES = {
    "mixed_with_padding": ([0, 130, 200], [300, 77, 0], 800, 2, 128),
    "tile_boundaries": ([5, 64, 128, 129, 127], [123, 64, 1, 127, 129], 1100, 3, 128),
    "single_token": ([0], [1], 8, 1, 128),
    # head_dim 64 runs its own kernels over the same lists
    "head_dim_64": ([0, 130, 200], [300, 77, 0], 800, 2, 64),
}


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("is_causal", [False, True])
def test_plan_matches_device_lists_bitwise(case, is_causal):
    prefix, causal, T, H, D = CASES[case]
    print(f"[plan] {case} is_causal={is_causal}", flush=True)
    b = make_batch(prefix, causal, T, H, D, seed=zlib.crc32(case.encode()) % 1000, device=DEV)
    ref = _fwd_bwd(b, is_causal, None)
    got = _fwd_bwd(b, is_causal, _plan_of(b, is_causal))
    for name, x, y in zip(("out", "lse", "out_lo", "dq", "dk", "dv"), ref, got):
        assert torch.equal(x, y), name


@pytest.mark.parametrize("cfg", [2, 4])
def test_plan_matches_on_benchmark_config(cfg):
    print(f"[plan] config {cfg}", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    ref = _fwd_bwd(b, False, None)
    # a plan built for is_causal=True only orders the lists differently
    for plan in (_plan_of(b, False), _plan_of(b, True)):
        got = _fwd_bwd(b, False, plan)
        for name, x, y in zip(("out", "lse", "out_lo", "dq", "dk", "dv"), ref, got):
            assert torch.equal(x, y), name


@pytest.mark.parametrize("seed", range(8))
def test_plan_matches_device_lists_on_random_packings(seed):
    """Seeded random packings (1-40 segments of 1-1500 rows, 1-4 heads, either
    is_causal): the host plan and the device-built lists give bitwise the same outputs."""
    rng = np.random.default_rng(5300 + seed)
    n = int(rng.integers(1, 41))
    L = np.exp(rng.uniform(0, np.log(1500), size=n)).astype(np.int64) + 1
    prefix = np.floor(rng.uniform(size=n) * (L + 1)).astype(np.int64)
    causal = L - prefix
    T = int(L.sum()) + int(rng.integers(0, 100))
    H = int(rng.integers(1, 5))
    is_causal = bool(rng.integers(0, 2))
    print(f"[plan] random{seed} n={n} T={T} H={H} is_causal={is_causal}", flush=True)
    b = make_batch(prefix, causal, T, H, 128, seed=5300 + seed, device=DEV)
    ref = _fwd_bwd(b, is_causal, None)
    got = _fwd_bwd(b, is_causal, _plan_of(b, is_causal))
    for name, x, y in zip(("out", "lse", "out_lo", "dq", "dk", "dv"), ref, got):
        assert torch.equal(x, y), name


def test_plan_for_other_metadata_is_rejected(monkeypatch):
    b = make_batch([10, 20], [30, 40], 128, 2, 128, seed=9, device=DEV)
    q = b.q.detach().clone().requires_grad_()
    # a plan of another size: rejected on the host before any launch
    big = make_batch([3] * 40, [2] * 40, 256, 2, 128, seed=9, device=DEV)
    with pytest.raises(RuntimeError, match="plan"):
        flash_attn_varlen_prefixlm(q, b.k, b.v, False, **b.seq_info, plan=_plan_of(big, False))
    # a plan of the same size built from other metadata: caught by the checking mode,
    # which rebuilds the plan from the call's metadata
    other = make_batch([10, 20, 5], [30, 40, 3], 128, 2, 128, seed=9, device=DEV)
    stale = _plan_of(other, False)
    assert stale.numel() == _plan_of(b, False).numel()
    monkeypatch.setattr(op, "_CHECK_METADATA", True)
    with pytest.raises(RuntimeError, match="plan does not match"):
        flash_attn_varlen_prefixlm(q, b.k, b.v, False, **b.seq_info, plan=stale)
    flash_attn_varlen_prefixlm(q, b.k, b.v, False, **b.seq_info, plan=_plan_of(b, False))


def test_more_segments_than_the_list_kernel_stages():
    """3000 segments, more than the device list builder stages in LDS (2048): its other
    path (each thread walking its own segments, and the stored-dS bases scanned in
    chunks of segments per thread) gives bitwise the plan's outputs, and both meet the
    parity bar against the fp32 oracle."""
    from test_gpu_parity import full_check
    rng = np.random.default_rng(17)
    L = rng.integers(1, 25, size=3000)
    p = np.floor(rng.uniform(0, 1, size=3000) * L).astype(np.int64)
    print("[plan] 3000 segments", flush=True)
    b = make_batch(p, L - p, int(L.sum()) + 37, 2, 128, seed=17, device=DEV)
    ref = _fwd_bwd(b, False, None)
    got = _fwd_bwd(b, False, _plan_of(b, False))
    for name, x, y in zip(("out", "lse", "out_lo", "dq", "dk", "dv"), ref, got):
        assert torch.equal(x, y), name
    full_check(b, tag="segments3000")
