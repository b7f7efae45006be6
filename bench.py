"""Benchmark: packed varlen PrefixLM attention forward + backward on one MI355X.

A step is one forward and one backward of ``flash_attn_varlen_prefixlm`` (through
its autograd path, gradients for q, k and v) over one synthetic packed batch whose
inputs already sit in HBM. The batch's work-list plan is built on the host before
the timed region, as the data loader would (``--no-plan``: the calls build their
work lists on the device instead). Default workload = config 2 (16384 packed tokens, log-normal segments,
16 heads x d128, bf16). Throughput counts only attended (query, key) pairs:
useful FLOPs = (4 + 10) * D * H * sum_seg N.

Prints one JSON line. Extra fields: per-direction times, the roofline of the
dominant kernel (per-launch HIP-event timing inside the timed region) and the
CPU baseline (the fp32 oracle's SDPA path on the host, same workload, bounded).

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--config 2]

``--workload stack`` instead times forward + backward of the config-5 HRM stack
(hidden 2048, 16 x d128, SwiGLU 5632, 2 H x 2 L cycles, ``--layers`` per module,
bf16, random weights, config-2 segmentation) three ways: the attention layer as the
reference composes it (PyTorch RoPE, the op, PyTorch gating), the fused layer, and
the fused layer with the SwiGLU / RMSNorm kernels; prints one JSON line with all three.

``--workload decode`` times one decode step of the KV-cache attention
(``flash_attn_with_kvcache``, S = 1, ``--batch`` rows x 16 heads x d128, caches of
``--cache-len`` keys): HBM-bound, reported in GB/s of cache read against 8 TB/s.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "hrm-text_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "PrefixLM varlen attn fwd+bwd useful TFLOP/s + % bf16 MFMA peak, 1 GPU"
PEAK_TFLOPS = 2500.0          # MI355X dense bf16 MFMA, published
HBM_GBPS = 8000.0
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-plan", action="store_true", help="build the work lists on the device per call")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--workload", choices=("attn", "stack", "decode"), default="attn")
    ap.add_argument("--batch", type=int, default=64, help="decode batch rows (decode workload)")
    ap.add_argument("--cache-len", type=int, default=4096, help="keys per cache row (decode workload)")
    ap.add_argument("--layers", type=int, default=8, help="layers per H/L module (stack workload)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (for scaling rocprof byte counters)")
    return ap.parse_args()


def calibrate_copy():
    """A plain device-to-device copy of exactly 256 MiB, five times. rocprofv3's
    FETCH_SIZE / WRITE_SIZE for this kernel divided by 256 MiB gives the factor that
    converts the counters into bytes for the attention kernels."""
    import torch
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "launches": 5}))


def cpu_baseline(batch, budget_s):
    """fp32 SDPA (MATH backend) forward + closed-form backward of the oracle on the
    host cores, segment by segment in batch order until the time budget is spent."""
    import torch
    from oracle.prefixlm_oracle import attention_bwd, attention_fwd_sdpa
    from prefixlm.metadata import useful_flops

    q, k, v, do = (t.detach().cpu().float() for t in (batch.q, batch.k, batch.v, batch.dout))
    H, D = q.shape[1], q.shape[2]
    flops = 0
    done = 0
    cs = 0
    segs = []
    for p, c in zip(batch.prefix.tolist(), batch.causal.tolist()):
        segs.append((cs, p, p + c))
        cs += p + c
    t0 = time.perf_counter()
    for (cs, p, L) in segs:
        attention_fwd_sdpa(q, k, v, [(cs, p, L)])
        attention_bwd(q, k, v, do, [(cs, p, L)])
        flops += useful_flops([p], [L - p], H, D)
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{done}/{len(segs)} segments of the same batch ({sum(s[2] for s in segs[:done])} "
                  f"tokens), fp32 SDPA MATH forward + closed-form backward, {dt:.1f} s",
    }


def bench_stack(args):
    """Config-5 stack forward + backward: PyTorch elementwise ops and the unfused op, the
    fused attention layer, and the fused layer with the SwiGLU / RMSNorm kernels."""
    import torch
    from prefixlm import build_plan, flash_attn_varlen_prefixlm, fused_attention_layer
    from prefixlm.hrm_stack import FusedLayer, HRMStack, HRMStackConfig, packed_position_ids
    from prefixlm.metadata import useful_entries
    from prefixlm.synth import metadata_tensors, segments_for_config

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    prefix, causal = segments_for_config(5)
    T = 16384
    st, ss = metadata_tensors(prefix, causal, T, dev)
    seq = {**st, **ss, "plan": torch.from_numpy(build_plan(st, ss)).to(dev)}
    pos = packed_position_ids(prefix, causal, T, dev)
    cfg = HRMStackConfig(layers_per_module=args.layers)
    model = HRMStack(cfg).init_weights(1005).to(dev, torch.bfloat16)
    g = torch.Generator(device="cpu").manual_seed(1005)
    x = torch.randn(T, cfg.hidden_size, generator=g).to(dev, torch.bfloat16).requires_grad_()
    dout = torch.randn(T, cfg.hidden_size, generator=g).to(dev, torch.bfloat16)
    params = [x] + list(model.parameters())

    def step(attn):
        out = model(x, pos, attn, seq)
        torch.autograd.grad(out, params, dout)

    res = {}
    for name, attn, fused_ew in (("unfused", flash_attn_varlen_prefixlm, False),
                                 ("fused", FusedLayer(fused_attention_layer), False),
                                 ("fused_all", FusedLayer(fused_attention_layer), True)):
        model.cfg.fused_elementwise = fused_ew
        for _ in range(args.warmup):
            step(attn)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step(attn)
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / args.steps
    calls = (cfg.H_cycles * (cfg.L_cycles + 1)) * args.layers
    attn_flops = calls * 14 * 128 * cfg.num_heads * useful_entries(prefix, causal)
    print(json.dumps({
        "metric": "config-5 HRM stack fwd+bwd ms per step (attention layer and elementwise ops fused)",
        "value": round(res["fused_all"], 3), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"cfg5 stack: {T} tokens, hidden 2048, 16 heads x d128, FFN 5632, "
                               f"2Hx2L cycles, {args.layers} layers per module, random init (seed 1005)",
                   "attention_calls_per_step": calls,
                   "attention_useful_tflop_per_step": round(attn_flops / 1e12, 3)},
        "ms_per_step_unfused": round(res["unfused"], 3),
        "ms_per_step_fused": round(res["fused"], 3),
        "ms_per_step_fused_all": round(res["fused_all"], 3),
        "saved_ms_per_attention_call": round((res["unfused"] - res["fused"]) / calls, 4),
    }), flush=True)


def bench_decode(args):
    """One decode step: append one k, v row per batch row, attend all cached keys."""
    import torch
    from prefixlm import flash_attn_with_kvcache

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, Lc = args.batch, 16, 128, args.cache_len
    g = torch.Generator(device="cuda").manual_seed(7)
    mk = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)  # noqa: E731
    q, k, v = mk(B, 1, H, D), mk(B, 1, H, D), mk(B, 1, H, D)
    kc, vc = mk(B, Lc, H, D), mk(B, Lc, H, D)
    lens = torch.full((B,), Lc - 1, dtype=torch.int32, device=dev)   # the step fills the last row

    def step():
        return flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=lens)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = B * H * Lc * D * 2 * 2          # every cached key and value read once
    gbps = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "KV-cache decode attention step, GB/s of cache read", "value": round(gbps, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"decode: batch {B}, 1 query, 16 heads x d128, {Lc} cached keys per row"},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_GBPS, 4), "traffic": None},
    }), flush=True)


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention op has no cross-GPU communication: each GPU attends over its own "
              "packed micro-batch, so N GPUs run N independent copies of this workload)",
              file=sys.stderr)
        sys.exit(2)

    if args.workload == "decode":
        if args.steps == 100 and args.warmup == 10:
            args.steps, args.warmup = 50, 5
        bench_decode(args)
        return
    if args.workload == "stack":
        if args.steps == 100 and args.warmup == 10:   # the attention-op defaults are too long here
            args.steps, args.warmup = 10, 2
        bench_stack(args)
        return

    import torch
    from prefixlm import _capi, build_plan, flash_attn_varlen_prefixlm
    from prefixlm.metadata import useful_entries
    from prefixlm.synth import make_config_batch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b = make_config_batch(args.config, device=dev, gen_device="cuda")
    T, H, D = b.q.shape
    n_useful = useful_entries(b.prefix, b.causal)
    f_fwd = 4 * D * H * n_useful
    f_bwd = 10 * D * H * n_useful
    q, k, v = (t.detach().clone().requires_grad_() for t in (b.q, b.k, b.v))
    seq = dict(b.seq_info)
    if not args.no_plan:
        seq["plan"] = torch.from_numpy(build_plan(b.seq_tensors, b.seq_scalars)).to(dev)

    def fwd():
        return flash_attn_varlen_prefixlm(q, k, v, False, **seq)

    def step():
        # gradients w.r.t. q, k, v through the autograd path; torch.autograd.grad
        # returns them instead of accumulating into leaf .grad buffers (in the model
        # q, k, v are intermediate activations, so nothing accumulates there)
        out = fwd()
        torch.autograd.grad(out, (q, k, v), b.dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # forward-only and backward-only splits (untimed for the headline value)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_split = max(5, args.steps // 4)
    e0.record()
    for _ in range(n_split):
        with torch.no_grad():
            fwd()
    e1.record()
    torch.cuda.synchronize()
    fwd_ms = e0.elapsed_time(e1) / n_split

    # headline: K full steps, per-kernel HIP events recorded around every launch
    _capi.timing_read()
    _capi.timing_enable(True)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    _capi.timing_enable(False)
    ms = start.elapsed_time(end) / args.steps
    kt = _capi.timing_read()

    value = (f_fwd + f_bwd) / (ms * 1e-3) / 1e12
    # algorithmic FLOPs of each MFMA kernel over the attended pairs: forward S and PV
    # (2 products), dK/dV kernel S, dP, dV, dK (4), dQ kernel S, dP, dQ (3; S and dP
    # are recomputed there, so the backward executes 7 products for the useful 5)
    kflops = {"fwd": f_fwd, "bwd_dkdv": 8 * D * H * n_useful, "bwd_dq": 6 * D * H * n_useful}
    avg = {k: kt[k][0] / max(1, kt[k][1]) for k in kflops}
    dom = max(avg, key=avg.get)
    dom_ms, dom_flops = avg[dom], kflops[dom]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        try:
            traffic = json.load(open(PROFILE_TRAFFIC)).get(f"cfg{args.config}", {}).get(dom)
        except (ValueError, OSError):
            traffic = None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(b, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"cfg{args.config}: {T} packed tokens, {len(b.prefix)} segments, "
                        f"{H} heads x d{D}, PrefixLM fwd+bwd (seed {1000 + args.config})",
            "tokens": T, "heads": H, "head_dim": D, "segments": int(len(b.prefix)),
            "useful_pairs_per_head": int(n_useful),
            "useful_tflop_per_step": round((f_fwd + f_bwd) / 1e12, 4),
            "work_lists": "device" if args.no_plan else "host plan",
        },
        "pct_of_peak": round(100.0 * value / PEAK_TFLOPS, 2),
        "fwd_ms": round(fwd_ms, 4),
        "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 2),
        "bwd_ms_est": round(ms - fwd_ms, 4),
        "kernel_avg_ms": {name: round(t / n, 4) for name, (t, n) in kt.items() if n},
        "kernel_tflops": {k: round(kflops[k] / (avg[k] * 1e-3) / 1e12, 1) for k in kflops if avg[k] > 0},
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
