"""GPU parity: the HIP kernels (through the C ABI and the torch op) against the
fp32 oracle and the fp64 golden vectors.

Tolerances (stated for the path): O, dQ, dK, dV within max-abs 2e-2 and mean-abs
2e-3 of the fp32 oracle evaluated on the same bf16 inputs; LSE within 1e-3
(max-abs). Rows past total_seqlen must be exactly zero.
"""
import ctypes
import os
import zlib

import numpy as np
import pytest
import torch

from oracle.prefixlm_oracle import attention_bwd, attention_fwd
from prefixlm import _capi, flash_attn_varlen_prefixlm, op
from prefixlm.synth import make_batch, make_config_batch, metadata_tensors

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
MAX_ABS, MEAN_ABS, LSE_ABS = 2e-2, 2e-3, 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def segs_of(prefix, causal):
    out, cs = [], 0
    for p, c in zip(prefix, causal):
        out.append((cs, int(p), int(p) + int(c)))
        cs += int(p) + int(c)
    return out


def run_fwd_bwd(b, is_causal=False, scale=None, q=None, k=None, v=None):
    q = (b.q if q is None else q).detach().clone().requires_grad_()
    k = (b.k if k is None else k).detach().clone().requires_grad_()
    v = (b.v if v is None else v).detach().clone().requires_grad_()
    out = flash_attn_varlen_prefixlm(q, k, v, is_causal, **b.seq_info, softmax_scale=scale)
    out.backward(b.dout)
    torch.cuda.synchronize()
    return out.detach(), q.grad, k.grad, v.grad


def compare(name, got, ref, total, tag=""):
    """Max-abs and mean-abs error of a bf16 output against the fp32 oracle. Printed with
    them: the bf16 rounding floor at the max-error element, |bf16(ref) - ref| (what an
    exact kernel whose output is rounded to bf16 would still show there), and the
    kernel's own share, |got - bf16(ref)| in units of that element's bf16 ulp."""
    g = got.float()
    err = (g[:total] - ref[:total]).abs()
    mx = err.max().item() if err.numel() else 0.0
    mean = err.mean().item() if err.numel() else 0.0
    refmax = ref[:total].abs().max().item() if err.numel() else 0.0
    floor, ulps = 0.0, 0.0
    if err.numel():
        i = int(err.argmax())
        r = ref[:total].reshape(-1)[i]
        rb = r.to(torch.bfloat16).float()
        floor = (rb - r).abs().item()
        ulp = torch.ldexp(torch.ones_like(rb), torch.frexp(rb).exponent - 8).item() if rb != 0 else 2.0 ** -133
        ulps = (g[:total].reshape(-1)[i] - rb).abs().item() / ulp
    print(f"[parity] {tag} {name}: max_abs={mx:.3e} mean_abs={mean:.3e} max|ref|={refmax:.3f} "
          f"floor={floor:.3e} kernel_ulps={ulps:.0f}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{tag} {name}: max {mx:.3e} mean {mean:.3e}"
    if total < got.shape[0]:
        assert (got[total:] == 0).all(), f"{tag} {name}: padding rows not zero"


def full_check(b, is_causal=False, scale=None, tag=""):
    segs = segs_of(b.prefix, b.causal)
    total = int(b.seq_scalars["total_seqlen"])
    out, dq, dk, dv = run_fwd_bwd(b, is_causal, scale)
    ref_o, ref_lse = attention_fwd(b.q, b.k, b.v, segs, is_causal, scale)
    compare("out", out, ref_o, total, tag)
    del ref_o
    sc = scale if scale is not None else 1.0 / np.sqrt(b.q.shape[-1])
    _, lse, _, _ = op.varlen_fwd(b.q, b.k, b.v, is_causal, *b.seq_info.values(), float(sc))
    lerr = (lse[:, :total] - ref_lse[:, :total]).abs().max().item() if total else 0.0
    print(f"[parity] {tag} lse: max_abs={lerr:.3e}", flush=True)
    assert lerr <= LSE_ABS
    if total < lse.shape[1]:
        assert torch.isinf(lse[:, total:]).all() and (lse[:, total:] < 0).all()
    del ref_lse
    ref = attention_bwd(b.q, b.k, b.v, b.dout, segs, is_causal, scale)
    for name, got, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        compare(name, got, r, total, tag)


@pytest.mark.parametrize("name", ["d128_prefixlm"])
def test_golden_vectors(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    T = int(z["num_tokens"])
    st, ss = metadata_tensors(z["prefix_lens"], z["causal_lens"], T, DEV)

    class B:
        pass
    b = B()
    b.q, b.k, b.v, b.dout = (torch.from_numpy(z[n]).to(DEV, torch.bfloat16) for n in ("q", "k", "v", "dout"))
    b.seq_info = {**st, **ss}
    causal = bool(z["is_causal"])
    out, dq, dk, dv = run_fwd_bwd(b, causal)
    total = int(ss["total_seqlen"])
    for n, got in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        compare(n, got, torch.from_numpy(z[n]).to(DEV), total, name)
    _, lse, _, _ = op.varlen_fwd(b.q, b.k, b.v, causal, *b.seq_info.values(), 1.0 / np.sqrt(128))
    assert (lse[:, :total] - torch.from_numpy(z["lse"]).to(DEV)[:, :total]).abs().max().item() <= LSE_ABS


EDGE = {
    "single_token": ([0], [1], 8, 1),
    "prefix_only_token": ([1], [0], 8, 1),
    "mixed_with_padding": ([0, 130, 200], [300, 77, 0], 800, 2),
    "tile_boundaries": ([5, 64, 128, 129, 127], [123, 64, 1, 127, 129], 1100, 3),
    # prefix ends and segment ends on both sides of 32-key tile edges (forward tiles)
    "key_tile_32_edges": ([31, 32, 33, 96, 0, 97], [1, 32, 63, 33, 95, 32], 700, 2),
    "long_prefix_only": ([4096], [0], 4200, 1),
    "long_causal_only": ([0], [2000], 2048, 2),
    "all_suffix_empty": ([100, 57, 33, 300], [0, 0, 0, 0], 512, 2),
    "prefix_over_tiles": ([700, 33], [900, 1400], 3040, 2),
    # one long segment among short ones: a 9-tile causal segment, and a long
    # prompt-heavy segment whose last query tiles carry the longest key loops
    "long_causal_among_short": ([0] + [40] * 8, [1152] + [30] * 8, 2048, 2),
    "long_prompt_among_short": ([3600] + [100] * 30, [496] + [28] * 30, 8192, 2),
}


@pytest.mark.parametrize("case", sorted(EDGE))
def test_edge_cases(case):
    prefix, causal, T, H = EDGE[case]
    b = make_batch(prefix, causal, T, H, 128, seed=zlib.crc32(case.encode()) % 1000, device=DEV)
    full_check(b, tag=case)


@pytest.mark.parametrize("case", ["mixed_with_padding", "tile_boundaries"])
def test_is_causal_flag(case):
    prefix, causal, T, H = EDGE[case]
    b = make_batch(prefix, causal, T, H, 128, seed=3, device=DEV)
    full_check(b, is_causal=True, tag=case + "/causal")


@pytest.mark.parametrize("D", [128, 64])
def test_out_lo_residual_codes(D):
    """out_lo holds int8 codes q with out + q 2^(e-16) the fp32 O (out = m 2^e, m in
    [0.5, 1)): the decoded value lies within half of out's bf16 ulp of out, sits closer to
    the fp64 oracle than out itself, and the padding rows' codes are 0."""
    prefix, causal, T, H = [0, 130, 200, 37], [300, 77, 0, 260], 1100, 3
    b = make_batch(prefix, causal, T, H, D, seed=11, device=DEV)
    total = int(sum(prefix) + sum(causal))
    sc = 1.0 / np.sqrt(D)
    out, _, lo, _ = op.varlen_fwd(b.q, b.k, b.v, False, *b.seq_info.values(), float(sc))
    torch.cuda.synchronize()
    assert lo.dtype == torch.int8 and tuple(lo.shape) == (T, H, D)
    o = out.float()
    e = torch.frexp(o).exponent
    dec = o + lo.float() * torch.ldexp(torch.ones_like(o), e - 16)
    ulp = torch.ldexp(torch.ones_like(o), e - 8)
    assert ((dec - o).abs() <= ulp / 2).all()
    ref, _ = attention_fwd(b.q, b.k, b.v, segs_of(prefix, causal), False, sc)
    ref = ref.to(DEV)[:total]
    e_out = (o[:total] - ref).abs().mean().item()
    e_dec = (dec[:total] - ref).abs().mean().item()
    print(f"[parity] out_lo D={D}: mean |out - ref| {e_out:.3e}, mean |out + residual - ref| {e_dec:.3e}", flush=True)
    assert e_dec < 0.75 * e_out
    assert (lo[total:] == 0).all()


def test_softmax_scale_argument():
    b = make_batch([50, 0], [60, 90], 256, 2, 128, seed=4, device=DEV)
    full_check(b, scale=0.05, tag="scale0.05")


@pytest.mark.parametrize("m,D", [(2.0 ** 13, 128), (2.0 ** -8, 128), (2.0 ** 13, 64)])
def test_q_beyond_the_unscaled_fp16_range(m, D):
    """q' = m q, k' = k / m (m a power of two) leaves S, O and dS unchanged and scales
    dQ by 1/m and dK by m exactly. With max |q'| outside [2^-4, 2^14] the dK/dV kernel
    converts q to fp16 with a power-of-two scale instead of unscaled: the rescaled
    gradients must agree with the unscaled run's (which meets the parity bar) to about
    one bf16 ulp."""
    b = make_batch([40, 0, 150], [200, 90, 20], 512, 2, D, seed=12, device=DEV)
    base = run_fwd_bwd(b)
    q2 = (b.q.float() * m).to(torch.bfloat16)
    k2 = (b.k.float() / m).to(torch.bfloat16)
    assert torch.equal(q2.float() / m, b.q.float()) and torch.equal(k2.float() * m, b.k.float())
    got = run_fwd_bwd(b, q=q2, k=k2)
    assert torch.equal(got[0], base[0])
    for name, g, r in (("dq", got[1].float() * m, base[1]), ("dk", got[2].float() / m, base[2]),
                       ("dv", got[3].float(), base[3])):
        d = (g - r.float()).abs().max().item()
        print(f"[parity] q x {m:g} D={D} {name}: max |rescaled - base| = {d:.3e}", flush=True)
        assert d <= 1e-2, name


def test_many_short_segments():
    rng = np.random.default_rng(5)
    L = rng.integers(1, 41, size=60)
    p = np.floor(rng.uniform(0, 1, size=60) * L).astype(np.int64)
    b = make_batch(p, L - p, int(L.sum()) + 40, 2, 128, seed=5, device=DEV)
    full_check(b, tag="short60")


def test_empty_batch_all_padding():
    T, H, D = 64, 2, 128
    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v, do = (torch.randn((T, H, D), generator=g).to(DEV, torch.bfloat16) for _ in range(4))
    seq = {n: torch.zeros(T, dtype=torch.int32, device=DEV) for n in ("prefix_lens", "causal_lens", "cu_seqlens")}
    for n in ("total_seqlen", "numseqs", "max_seqlen_prefix", "max_seqlen_causal", "max_seqlen_all"):
        seq[n] = torch.tensor(0)
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    out = flash_attn_varlen_prefixlm(qq, kk, vv, False, **seq)
    out.backward(do)
    torch.cuda.synchronize()
    for t in (out, qq.grad, kk.grad, vv.grad):
        assert (t == 0).all()


def test_strided_v_view_matches_contiguous():
    """v as a view of a fused [T, 4H, D] projection (reference models/layers.py:131-135)."""
    prefix, causal, T, H = [40, 0, 150], [200, 90, 20], 512, 2
    b = make_batch(prefix, causal, T, H, 128, seed=6, device=DEV)
    fused = torch.cat([b.q, b.q, b.k, b.v], dim=1)           # gate, q, k, v
    _, q_view, k_view, v_view = fused.split((H, H, H, H), dim=1)
    assert v_view.stride(0) == 4 * H * 128 and not v_view.is_contiguous()
    ref = run_fwd_bwd(b)
    got = run_fwd_bwd(b, q=q_view, k=k_view, v=v_view)
    for r, g in zip(ref, got):
        assert torch.equal(r, g) or (r.float() - g.float()).abs().max().item() < 1e-2
    assert torch.equal(ref[0], got[0])


@pytest.mark.parametrize("D", [128, 64])
def test_forward_and_backward_are_bitwise_deterministic(D):
    # no kernel accumulates with floating-point atomics, so dq is reproducible too
    b = make_batch([300, 0, 64], [500, 700, 200], 1800, 2, D, seed=7, device=DEV)
    a1 = run_fwd_bwd(b)
    a2 = run_fwd_bwd(b)
    for x, y in zip(a1, a2):
        assert torch.equal(x, y)


def test_inconsistent_metadata_is_reported(monkeypatch):
    b = make_batch([10, 20], [30, 40], 128, 2, 128, seed=8, device=DEV)
    seq = dict(b.seq_info)
    cu = seq["cu_seqlens"].clone()
    cu[1] += 5                                   # segment 0 no longer ends where it says
    seq["cu_seqlens"] = cu
    monkeypatch.setattr(op, "_CHECK_METADATA", True)
    with pytest.raises(RuntimeError, match="inconsistent metadata"):
        op.varlen_fwd(b.q, b.k, b.v, False, *seq.values(), 0.088)
    torch.cuda.synchronize()
    # the consistent batch passes the same check
    op.varlen_fwd(b.q, b.k, b.v, False, *b.seq_info.values(), 0.088)


def test_capi_direct_call_matches_op():
    """Drive prefixlm_fwd through ctypes exactly as an FFI caller would."""
    b = make_batch([33, 0], [70, 50], 200, 2, 128, seed=9, device=DEV)
    lib = _capi.load()
    T, H, D = b.q.shape
    total, nseq = int(b.seq_scalars["total_seqlen"]), int(b.seq_scalars["numseqs"])
    out = torch.empty_like(b.q)
    lse = torch.empty((H, T), dtype=torch.float32, device=DEV)
    ws_bytes = lib.prefixlm_fwd_workspace_size(T, H, D, total, nseq)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    P = lambda t: t.data_ptr()
    st = b.seq_tensors
    sc = b.seq_scalars
    a = _capi.FwdArgs(
        q=P(b.q), k=P(b.k), v=P(b.v), out=P(out), out_lo=None, lse=P(lse),
        q_stride_t=H * D, q_stride_h=D, k_stride_t=H * D, k_stride_h=D,
        v_stride_t=H * D, v_stride_h=D, out_stride_t=H * D, out_stride_h=D,
        out_lo_stride_t=0, out_lo_stride_h=0,
        prefix_lens=P(st["prefix_lens"]), causal_lens=P(st["causal_lens"]),
        cu_seqlens=P(st["cu_seqlens"]), meta_len=T, num_tokens=T, num_heads=H, head_dim=D,
        total_seqlen=total, numseqs=nseq, max_seqlen_prefix=int(sc["max_seqlen_prefix"]),
        max_seqlen_causal=int(sc["max_seqlen_causal"]), max_seqlen_all=int(sc["max_seqlen_all"]),
        is_causal=0, softmax_scale=float(1.0 / np.sqrt(D)), workspace=P(ws), workspace_bytes=ws_bytes)
    rc = lib.prefixlm_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _capi.last_error()
    err = ctypes.c_int32(-1)
    assert lib.prefixlm_check_workspace(ctypes.c_void_p(ws.data_ptr()),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                        ctypes.byref(err)) == 0 and err.value == 0
    ref, _, _, _ = op.varlen_fwd(b.q, b.k, b.v, False, *b.seq_info.values(), 1.0 / np.sqrt(D))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("cfg", [2, 4, 3])
def test_benchmark_configs(cfg):
    print(f"[parity] config {cfg}: generating", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    full_check(b, tag=f"cfg{cfg}")


@pytest.mark.parametrize("cfg", [2, 4])
def test_benchmark_configs_is_causal(cfg):
    """is_causal=True on the benchmark packings: the reference's pass 1 then runs causal
    too (models/flash_attention_prefixlm_v2.py:115-121), so every segment is plain
    causal."""
    print(f"[parity] config {cfg} is_causal: generating", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    full_check(b, is_causal=True, tag=f"cfg{cfg}/causal")


@pytest.mark.parametrize("heads", [12, 10])
def test_config2_segmentation_model_head_counts(heads):
    """The reference's model sizes use 12 (XL) and 10 (L) heads
    (config/arch/size/XL.yaml, L.yaml): config 2's segmentation at those head counts.
    With H not a multiple of 8 a head's workgroups spread over several XCDs."""
    from prefixlm.synth import CONFIG_SHAPES, segments_for_config
    T, _, D = CONFIG_SHAPES[2]
    prefix, causal = segments_for_config(2)
    print(f"[parity] config 2 segmentation, {heads} heads: generating", flush=True)
    b = make_batch(prefix, causal, T, heads, D, 1002, device=DEV, gen_device="cuda")
    full_check(b, tag=f"cfg2/h{heads}")


@pytest.mark.parametrize("heads,D", [(32, 128), (24, 64), (20, 128)])
def test_more_heads_than_xcds(heads, D):
    """More heads than XCDs: 32 and 24 give each XCD several whole heads (head x, x + 8,
    ...), 20 two whole heads and a share of the remaining four; four segments with
    prefix-only, causal-only, mixed and padding rows."""
    prefix, causal, T = [0, 130, 200, 77], [300, 77, 0, 260], 1100
    print(f"[parity] {heads} heads x d{D}: generating", flush=True)
    b = make_batch(prefix, causal, T, heads, D, seed=heads * 7 + D, device=DEV)
    full_check(b, tag=f"h{heads}/d{D}")


@pytest.mark.parametrize("case", ["mixed_with_padding", "tile_boundaries", "prefix_over_tiles"])
def test_head_dim_64(case):
    """head_dim 64: forward and backward kernels of its own (half the operand registers,
    384-byte wide LDS rows in the backward)."""
    prefix, causal, T, H = EDGE[case]
    b = make_batch(prefix, causal, T, H, 64, seed=zlib.crc32(case.encode()) % 1000 + 64, device=DEV)
    full_check(b, tag=case + "/d64")


def test_head_dim_64_config1_shape():
    """Config 1's shape (4096 tokens, 8 heads x 64), in bf16 on the GPU."""
    b = make_config_batch(1, device=DEV, dtype=torch.bfloat16, gen_device="cuda")
    full_check(b, tag="cfg1/d64")


def _random_packing(rng):
    """A packed batch of 1-12 segments: lengths from 1 to 700 (log-uniform, so short
    segments are common), prefixes anywhere in [0, L] with extra weight on 0 and L,
    and 0-300 padding rows."""
    n = int(rng.integers(1, 13))
    L = np.exp(rng.uniform(0, np.log(700), size=n)).astype(np.int64) + 1
    u = rng.uniform(size=n)
    p = np.where(u < 0.15, 0, np.where(u > 0.85, L, np.floor(rng.uniform(size=n) * (L + 1)))).astype(np.int64)
    p = np.minimum(p, L)
    return p, L - p, int(L.sum()) + int(rng.integers(0, 301))


@pytest.mark.parametrize("seed", range(48))
def test_random_packings(seed):
    """Seeded random packings, head counts 1-5, head_dim 128 or (one in four) 64 and
    either is_causal value, against the oracle at the same bar (the kernels' tile, mask
    and list logic on shapes nobody chose by hand)."""
    rng = np.random.default_rng(7000 + seed)
    prefix, causal, T = _random_packing(rng)
    H = int(rng.integers(1, 6))
    is_causal = bool(rng.integers(0, 2))
    D = 64 if seed % 4 == 3 else 128
    tag = f"random{seed} n={len(prefix)} T={T} H={H} D={D} causal={is_causal}"
    print(f"[parity] {tag}: L={(prefix + causal).tolist()} p={prefix.tolist()}", flush=True)
    b = make_batch(prefix, causal, T, H, D, seed=7000 + seed, device=DEV)
    full_check(b, is_causal=is_causal, tag=tag)


def _random_long_packing(rng):
    """2-6 segments of 300-4096 rows (log-uniform) with prefixes anywhere in [0, L] and
    0-200 padding rows: many key tiles per segment, so the persistent dK/dV kernel's
    item loop, the dS block layout and the forward's long key loops meet shapes nobody
    chose by hand."""
    n = int(rng.integers(2, 7))
    L = np.exp(rng.uniform(np.log(300), np.log(4096), size=n)).astype(np.int64)
    p = np.floor(rng.uniform(size=n) * (L + 1)).astype(np.int64)
    p = np.minimum(p, L)
    return p, L - p, int(L.sum()) + int(rng.integers(0, 201))


@pytest.mark.parametrize("seed", range(6))
def test_random_long_packings(seed):
    rng = np.random.default_rng(9100 + seed)
    prefix, causal, T = _random_long_packing(rng)
    H = int(rng.integers(2, 9))
    is_causal = seed % 3 == 2
    tag = f"random_long{seed} n={len(prefix)} T={T} H={H} causal={is_causal}"
    print(f"[parity] {tag}: L={(prefix + causal).tolist()} p={prefix.tolist()}", flush=True)
    b = make_batch(prefix, causal, T, H, 128, seed=9100 + seed, device=DEV)
    full_check(b, is_causal=is_causal, tag=tag)
