"""The backward's two dQ paths on the GPU.

With a dS buffer (the default whenever the batch's buffer fits PREFIXLM_DS_MAX_BYTES)
the dK/dV kernel also stores dS and dQ is a streaming product over the stored dS; with
PREFIXLM_DS_MAX_BYTES=0 the dQ kernel recomputes S, P and dP. Both paths meet the
parity bar against the fp32 oracle (max-abs 2e-2, mean-abs 2e-3). dK and dV come from
the same kernel on both paths and must be bitwise equal; dQ differs by rounding only.
"""
import zlib

import pytest
import torch

from prefixlm import _capi, flash_attn_varlen_prefixlm, op
from prefixlm.synth import make_batch, make_config_batch
from test_gpu_parity import EDGE, full_check, run_fwd_bwd

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CASES = ["mixed_with_padding", "tile_boundaries", "prefix_over_tiles", "long_prompt_among_short"]


def _batch(case, D=128):
    prefix, causal, T, H = EDGE[case]
    return make_batch(prefix, causal, T, H, D, seed=zlib.crc32(case.encode()) % 1000 + D, device=DEV)


@pytest.mark.parametrize("case", CASES)
def test_recompute_path_parity(case, monkeypatch):
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", "0")
    full_check(_batch(case), tag=case + "/recompute")


def test_recompute_path_head_dim_64(monkeypatch):
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", "0")
    full_check(_batch("tile_boundaries", 64), tag="tile_boundaries/d64/recompute")


@pytest.mark.parametrize("cfg", [3, 4])
def test_recompute_path_benchmark_configs(cfg, monkeypatch):
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", "0")
    print(f"[ds] config {cfg} recompute: generating", flush=True)
    full_check(make_config_batch(cfg, device=DEV, gen_device="cuda"), tag=f"cfg{cfg}/recompute")


@pytest.mark.parametrize("case,D", [(c, 128) for c in CASES] + [("prefix_over_tiles", 64)])
def test_paths_agree(case, D, monkeypatch):
    b = _batch(case, D)
    T, H, _ = b.q.shape
    lib = _capi.load()
    sc = b.seq_scalars
    assert lib.prefixlm_bwd_ds_bytes(T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"])) > 0
    monkeypatch.delenv("PREFIXLM_DS_MAX_BYTES", raising=False)
    out_ds, dq_ds, dk_ds, dv_ds = run_fwd_bwd(b)
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", "0")
    out_rc, dq_rc, dk_rc, dv_rc = run_fwd_bwd(b)
    assert torch.equal(out_ds, out_rc)
    assert torch.equal(dk_ds, dk_rc) and torch.equal(dv_ds, dv_rc)
    diff = (dq_ds.float() - dq_rc.float()).abs().max().item()
    print(f"[ds] {case}/d{D}: dq paths differ by max-abs {diff:.3e}", flush=True)
    assert diff <= 1e-2


def test_ds_buffer_follows_the_cap(monkeypatch):
    b = _batch("mixed_with_padding")
    T, H, _ = b.q.shape
    lib = _capi.load()
    sc = b.seq_scalars
    n = lib.prefixlm_bwd_ds_bytes(T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"]))
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", str(n))
    p, nb, buf, _ = op._ds_arg(lib, T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"]), DEV)
    assert nb == n and buf is not None and buf.numel() == n
    monkeypatch.setenv("PREFIXLM_DS_MAX_BYTES", str(n - 1))
    p, nb, buf, _ = op._ds_arg(lib, T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"]), DEV)
    assert nb == 0 and buf is None and not p.value


@pytest.mark.parametrize("cfg", [2, 4])
def test_exact_plan_buffer_matches_the_bound(cfg, monkeypatch):
    """With a plan and its plan_ds_blocks the dS buffer holds exactly the attended blocks
    (0.54 GB on config 2, 0.60 GB on config 4, against 1.5 and 5.1 GB from the
    max_seqlen bound); the gradients are bitwise those of the bound-sized buffer with
    device-built lists and with the plan alone."""
    from prefixlm import plan_inputs
    monkeypatch.delenv("PREFIXLM_DS_MAX_BYTES", raising=False)
    print(f"[ds] config {cfg} exact buffer: generating", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    T, H, _ = b.q.shape
    sc = b.seq_scalars
    pi = plan_inputs(b.seq_tensors, sc, DEV)
    args = (T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"]))
    exact = op.ds_buffer_bytes(*args, plan_ds_blocks=pi["plan_ds_blocks"], device=DEV)
    bound = op.ds_buffer_bytes(*args, device=DEV)
    print(f"[ds] config {cfg}: exact {exact / 1e9:.3f} GB, bound {bound / 1e9:.3f} GB", flush=True)
    assert 0 < exact < bound
    assert exact <= {2: 0.6e9, 4: 0.7e9}[cfg]
    res = []
    for seq in (dict(b.seq_info), {**b.seq_info, "plan": pi["plan"]}, {**b.seq_info, **pi}):
        q, k, v = (t.detach().clone().requires_grad_() for t in (b.q, b.k, b.v))
        out = flash_attn_varlen_prefixlm(q, k, v, False, **seq)
        out.backward(b.dout)
        torch.cuda.synchronize()
        res.append((q.grad, k.grad, v.grad))
    for other in res[1:]:
        for x, y in zip(res[0], other):
            assert torch.equal(x, y)


def test_segment_longer_than_max_seqlen_all_is_reported(monkeypatch):
    """A segment longer than max_seqlen_all (which sizes the dS buffer without a plan) is
    inconsistent metadata: the checking mode raises instead of dropping dS blocks."""
    b = make_batch([10, 200], [30, 40], 320, 2, 128, seed=8, device=DEV)
    seq = dict(b.seq_info)
    seq["max_seqlen_all"] = torch.tensor(100, dtype=torch.int64)
    monkeypatch.setattr(op, "_CHECK_METADATA", True)
    out, lse, lo, qa = op.varlen_fwd(b.q, b.k, b.v, False, *b.seq_info.values(), 0.088)
    with pytest.raises(RuntimeError, match="inconsistent metadata"):
        op.varlen_bwd(b.q, b.k, b.v, False, b.dout, out, lse, lo, qa, *seq.values(), 0.088)
    torch.cuda.synchronize()
    op.varlen_bwd(b.q, b.k, b.v, False, b.dout, out, lse, lo, qa, *b.seq_info.values(), 0.088)
    torch.cuda.synchronize()


@pytest.mark.parametrize("D", [128, 64])
def test_zero_dout_with_v_beyond_fp16(D):
    """dO = 0 with |V| far above the fp16 range: the stored-dS scale over dO's scale is then
    1 whatever V is, so dP's V operand falls back to V's own safe scale (the dS values are
    rescaled before their store). Every gradient is exactly 0; with V converted at scale 1
    they would be NaN (inf * 0)."""
    b = _batch("mixed_with_padding", D)
    v = (b.v.float() * 2.0 ** 20).to(torch.bfloat16)
    q, k, vv = (t.detach().clone().requires_grad_() for t in (b.q, b.k, v))
    out = flash_attn_varlen_prefixlm(q, k, vv, False, **b.seq_info)
    out.backward(torch.zeros_like(out))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for name, g in (("dq", q.grad), ("dk", k.grad), ("dv", vv.grad)):
        assert torch.isfinite(g.float()).all() and (g == 0).all(), name
