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
PEAK_TFLOPS = 2516.6          # MI355X dense bf16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk/CU
HBM_GBPS = 8000.0
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prewarm-s", type=float, default=0.25,
                    help="seconds of untimed steps before the warmup steps (the GPU's clocks ramp up under "
                         "load; 0 turns it off)")
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-plan", action="store_true", help="build the work lists on the device per call")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra lines (other configs, head counts 12 and 10, the other work-list mode)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--workload", choices=("attn", "stack", "decode"), default="attn")
    ap.add_argument("--batch", type=int, default=64, help="decode batch rows (decode workload)")
    ap.add_argument("--cache-len", type=int, default=4096, help="keys per cache row (decode workload)")
    ap.add_argument("--layers", type=int, default=8, help="layers per H/L module (stack workload)")
    ap.add_argument("--bp-steps", type=int, default=2,
                    help="module calls that keep gradients (stack workload; the reference's default 2; "
                         "0 = all)")
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


def _host_info():
    """CPU model, counts and the thread count the baseline uses. The box's CPU share
    can be smaller than what os.cpu_count() reports (OMP_NUM_THREADS holds it on the
    GPU boxes), so the threads follow OMP_NUM_THREADS, else the affinity mask."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or affinity
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "threads": threads}


def cpu_baseline(batch, budget_s):
    """The oracle on the host cores (torch fp32, all usable threads):
    * value: config-2 fwd+bwd, fp32 SDPA (MATH) forward + closed-form backward,
      segment by segment in batch order until the time budget is spent;
    * c1: BASELINE config 1 (4096 tokens, 4 segments, 8 heads x d64), fp32 forward
      over the whole batch, median of 5 runs after 2 warm-ups."""
    import statistics
    import torch
    from oracle.prefixlm_oracle import attention_bwd, attention_fwd_sdpa
    from prefixlm.metadata import useful_flops
    from prefixlm.synth import make_config_batch

    info = _host_info()
    torch.set_num_threads(info["threads"])

    b1 = make_config_batch(1, device="cpu", dtype=torch.float32)
    segs1, cs = [], 0
    for p, c in zip(b1.prefix.tolist(), b1.causal.tolist()):
        segs1.append((cs, p, p + c))
        cs += p + c
    f1 = useful_flops(b1.prefix, b1.causal, b1.q.shape[1], b1.q.shape[2], fwd=True, bwd=False)
    times = []
    for i in range(7):
        t0 = time.perf_counter()
        attention_fwd_sdpa(b1.q, b1.k, b1.v, segs1)
        if i >= 2:
            times.append(time.perf_counter() - t0)
    t1 = statistics.median(times)

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
        "value": round(flops / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"config 2: {done}/{len(segs)} segments of the same batch ({sum(s[2] for s in segs[:done])} "
                  f"tokens), fp32 SDPA MATH forward + closed-form backward, {dt:.1f} s",
        **info,
        "c1_config1_fwd": {
            "value": round(f1 / t1 / 1e12, 4), "unit": "TFLOP/s", "ms": round(t1 * 1e3, 2),
            "sample": f"config 1: {len(segs1)} segments, {b1.q.shape[0]} tokens, 8 heads x d64, fp32 forward, "
                      "median of 5 after 2 warm-ups",
        },
    }


def _stack_setup(layers):
    """Config-5 HRM stack (random weights, seed 1005) on config-2 segmentation."""
    import torch
    from prefixlm import plan_inputs
    from prefixlm.hrm_stack import HRMStack, HRMStackConfig, packed_position_ids
    from prefixlm.synth import metadata_tensors, segments_for_config

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    prefix, causal = segments_for_config(5)
    T = 16384
    st, ss = metadata_tensors(prefix, causal, T, dev)
    seq = {**st, **ss, **plan_inputs(st, ss, dev)}
    pos = packed_position_ids(prefix, causal, T, dev)
    cfg = HRMStackConfig(layers_per_module=layers)
    model = HRMStack(cfg).init_weights(1005).to(dev, torch.bfloat16)
    g = torch.Generator(device="cpu").manual_seed(1005)
    x = torch.randn(T, cfg.hidden_size, generator=g).to(dev, torch.bfloat16)
    dout = torch.randn(T, cfg.hidden_size, generator=g).to(dev, torch.bfloat16)
    return dict(prefix=prefix, causal=causal, T=T, seq=seq, pos=pos, cfg=cfg, model=model, x=x, dout=dout)


def _timed_ms(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def stack_case(layers, steps, warmup, bp_steps=2):
    """BASELINE G5 in the default line: the config-5 stack with the fused attention layer
    and the SwiGLU / RMSNorm kernels; forward alone (no autograd) and the reference's
    training step (forward, then the backward of the last bp_steps module calls)."""
    import torch
    from prefixlm import fused_attention_layer
    from prefixlm.hrm_stack import FusedLayer
    from prefixlm.metadata import useful_entries

    s = _stack_setup(layers)
    model, cfg = s["model"], s["cfg"]
    model.cfg.fused_elementwise = True
    attn = FusedLayer(fused_attention_layer)
    params = list(model.parameters())
    bp = None if bp_steps <= 0 else bp_steps

    def fwd():
        with torch.no_grad():
            model(s["x"], s["pos"], attn, s["seq"], bp_steps=bp)

    def step():
        out = model(s["x"], s["pos"], attn, s["seq"], bp_steps=bp)
        torch.autograd.grad(out, params, s["dout"], allow_unused=True)

    fwd_ms = _timed_ms(fwd, steps, warmup)
    step_ms = _timed_ms(step, steps, warmup)
    calls = (cfg.H_cycles * (cfg.L_cycles + 1)) * layers
    n = useful_entries(s["prefix"], s["causal"])
    return {"fwd_ms": round(fwd_ms, 3), "fwd_bwd_ms": round(step_ms, 3), "layers_per_module": layers,
            "attention_calls": calls, "bp_steps": bp_steps,
            "fwd_attention_tflop": round(calls * 4 * 128 * cfg.num_heads * n / 1e12, 3),
            "workload": f"cfg5 stack: {s['T']} tokens, hidden 2048, 16 heads x d128, FFN 5632, 2Hx2L cycles, "
                        f"{layers} layers per module, random init (seed 1005), fused attention layer and "
                        "SwiGLU / RMSNorm kernels; parity in tests/test_gpu_stack.py"}


def bench_stack(args):
    """Config-5 stack forward + backward: PyTorch elementwise ops and the unfused op, the
    fused attention layer, and the fused layer with the SwiGLU / RMSNorm kernels."""
    import torch
    from prefixlm import flash_attn_varlen_prefixlm, fused_attention_layer
    from prefixlm.hrm_stack import FusedLayer
    from prefixlm.metadata import useful_entries

    s = _stack_setup(args.layers)
    prefix, causal, T, seq, pos, cfg, model, x, dout = (s[k] for k in ("prefix", "causal", "T", "seq", "pos", "cfg",
                                                                       "model", "x", "dout"))
    params = list(model.parameters())
    bp = None if args.bp_steps <= 0 else args.bp_steps
    l_grad, h_grad = model.grad_windows(bp)

    def step(attn):
        # the reference's recurrence: only the last bp_steps module calls keep gradients
        out = model(x, pos, attn, seq, bp_steps=bp)
        torch.autograd.grad(out, params, dout, allow_unused=True)

    res = {}
    for name, attn, fused_ew, fused_gemm in (("unfused", flash_attn_varlen_prefixlm, False, False),
                                             ("fused", FusedLayer(fused_attention_layer), False, False),
                                             ("fused_all", FusedLayer(fused_attention_layer), True, False),
                                             ("fused_gemm", FusedLayer(fused_attention_layer), True, True)):
        model.cfg.fused_elementwise = fused_ew
        model.cfg.fused_gemm = fused_gemm
        res[name] = _timed_ms(lambda: step(attn), args.steps, args.warmup)
    calls = (cfg.H_cycles * (cfg.L_cycles + 1)) * args.layers
    grad_calls = (len(l_grad) + len(h_grad)) * args.layers
    # every call runs the forward; only the calls inside the window run the backward
    attn_flops = (calls * 4 + grad_calls * 10) * 128 * cfg.num_heads * useful_entries(prefix, causal)
    print(json.dumps({
        "metric": "config-5 HRM stack fwd+bwd ms per step (attention layer and elementwise ops fused)",
        "value": round(res["fused_all"], 3), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"cfg5 stack: {T} tokens, hidden 2048, 16 heads x d128, FFN 5632, "
                               f"2Hx2L cycles, {args.layers} layers per module, random init (seed 1005), "
                               f"bp_steps {bp}",
                   "attention_calls_per_step": calls,
                   "attention_calls_with_backward": grad_calls,
                   "attention_useful_tflop_per_step": round(attn_flops / 1e12, 3)},
        "ms_per_step_unfused": round(res["unfused"], 3),
        "ms_per_step_fused": round(res["fused"], 3),
        "ms_per_step_fused_all": round(res["fused_all"], 3),
        "ms_per_step_fused_all_plus_norm_swiglu_gemm": round(res["fused_gemm"], 3),
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
    from prefixlm import _capi

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    head = _attn_case(args.config, None, args.steps, args.warmup, plan=not args.no_plan, timed_kernels=True,
                      prewarm_s=args.prewarm_s,
                      fwd_split=True)
    T, H, D, n_useful = head["T"], head["H"], head["D"], head["n_useful"]
    f_fwd, f_bwd = 4 * D * H * n_useful, 10 * D * H * n_useful
    ms = head["ms"]
    value = (f_fwd + f_bwd) / (ms * 1e-3) / 1e12
    kt = head["kernels"]
    # algorithmic FLOPs of each MFMA kernel over the attended pairs: forward S and PV
    # (2 products), dK/dV kernel S, dP, dV, dK (4), dQ kernel: dQ from the stored dS (1)
    # or S, dP, dQ when it recomputes (3; the backward then executes 7 products for the
    # useful 5)
    from prefixlm.op import ds_path_used
    sc = head["batch"].seq_scalars
    ds_path = ds_path_used(T, H, int(sc["numseqs"]), int(sc["max_seqlen_all"]))
    kflops = {"fwd": f_fwd, "bwd_dkdv": 8 * D * H * n_useful, "bwd_dq": (2 if ds_path else 6) * D * H * n_useful}
    avg = {k: kt[k][0] / max(1, kt[k][1]) for k in kflops}
    dom = max(avg, key=avg.get)
    dom_ms, dom_flops = avg[dom], kflops[dom]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    # HBM bytes per launch of the dominant kernel: not measured in this run (rocprofv3
    # --pmc cannot run inside it) but read from the committed profile summary of the
    # same workload and kernels
    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        try:
            traffic = json.load(open(PROFILE_TRAFFIC)).get(f"cfg{args.config}", {}).get(dom)
        except (ValueError, OSError):
            traffic = None

    extra = {}
    if not args.no_extra:
        # the same step with work lists built on the device per call (no host plan)
        other = _attn_case(args.config, None, max(10, args.steps // 2), 3, plan=args.no_plan,
                           prewarm_s=args.prewarm_s)
        extra["ms_per_step_" + ("host_plan" if args.no_plan else "device_lists")] = round(other["ms"], 4)
        cases = [(c, None) for c in (3, 4) if c != args.config] + [(args.config, 12), (args.config, 10)]
        for cfg, heads in cases:
            steps = {3: 5, 4: 20, 2: 20}[cfg]
            r = _attn_case(cfg, heads, steps, 2, plan=True, timed_kernels=True, prewarm_s=args.prewarm_s)
            key = f"cfg{cfg}" + (f"_h{heads}" if heads else "")
            extra[key] = _case_summary(r)
            del r
            torch.cuda.empty_cache()
        # BASELINE G5: the config-5 stack (8 layers per module, as in --workload stack)
        extra["cfg5_stack"] = stack_case(8, 5, 2)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(head["batch"], args.cpu_seconds)

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
            "workload": f"cfg{args.config}: {T} packed tokens, {head['segments']} segments, "
                        f"{H} heads x d{D}, PrefixLM fwd+bwd (seed {1000 + args.config})",
            "tokens": T, "heads": H, "head_dim": D, "segments": head["segments"],
            "useful_pairs_per_head": int(n_useful),
            "useful_tflop_per_step": round((f_fwd + f_bwd) / 1e12, 4),
            "work_lists": "device" if args.no_plan else "host plan",
            "dq_path": "stored dS" if ds_path else "recompute",
            "prewarm_s": args.prewarm_s,
            "prewarm_steps": head["prewarm_steps"],
        },
        "pct_of_peak": round(100.0 * value / PEAK_TFLOPS, 2),
        "peak_tflops": PEAK_TFLOPS,
        "fwd_ms": round(head["fwd_ms"], 4),
        "fwd_calls_timed": head["fwd_calls"],
        "fwd_tflops": round(f_fwd / (head["fwd_ms"] * 1e-3) / 1e12, 2),
        "bwd_ms_est": round(ms - head["fwd_ms"], 4),
        "hbm_floor_ms": round(_hbm_bytes(T, H, D) / (HBM_GBPS * 1e9) * 1e3, 4),
        "host_us_per_call": head["host_us"],
        "ms_per_step_with_kernel_events": round(head["ms_timed"], 4),
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
            "traffic_source": ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel on "
                               "this workload, scaled by a plain copy's counters; not measured in this run")
            if traffic is not None else None,
        },
        **extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _attn_case(cfg, heads, steps, warmup, plan=True, timed_kernels=False, fwd_split=False, prewarm_s=0.0):
    """Times `steps` fwd+bwd steps of the autograd path on config `cfg` (optionally
    with another head count on the same segmentation). The headline loop records no
    per-launch events; with `timed_kernels` a second loop of the same length runs with
    a per-kernel timer. Before the `warmup` steps, untimed steps run for `prewarm_s`
    seconds: the GPU's clocks ramp up over the first ~30 ms of load (a config-2 step
    takes 0.86 ms at steps 5-9 of a cold process, 0.71 ms from step 50 on)."""
    import torch
    from prefixlm import _capi, flash_attn_varlen_prefixlm, plan_inputs
    from prefixlm.metadata import useful_entries
    from prefixlm.synth import CONFIG_SHAPES, make_batch, make_config_batch, segments_for_config

    dev = torch.device("cuda:0")
    if heads is None:
        b = make_config_batch(cfg, device=dev, gen_device="cuda")
    else:
        T0, _, D0 = CONFIG_SHAPES[cfg]
        prefix, causal = segments_for_config(cfg)
        b = make_batch(prefix, causal, T0, heads, D0, 1000 + cfg, device=dev, gen_device="cuda",
                       k_scale=2.0 if cfg == 3 else 1.0)
    T, H, D = b.q.shape
    n_useful = useful_entries(b.prefix, b.causal)
    q, k, v = (t.detach().clone().requires_grad_() for t in (b.q, b.k, b.v))
    seq = dict(b.seq_info)
    if plan:
        seq.update(plan_inputs(b.seq_tensors, b.seq_scalars, dev))

    def fwd():
        return flash_attn_varlen_prefixlm(q, k, v, False, **seq)

    def step():
        # gradients w.r.t. q, k, v through the autograd path; torch.autograd.grad
        # returns them instead of accumulating into leaf .grad buffers (in the model
        # q, k, v are intermediate activations, so nothing accumulates there)
        out = fwd()
        torch.autograd.grad(out, (q, k, v), b.dout)

    def timed(fn, n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    n_pre = 0
    if prewarm_s > 0:
        step()                         # first-call costs (code objects, allocations) first
        torch.cuda.synchronize()
        n_pre = 1
        t_end = time.perf_counter() + prewarm_s
        while time.perf_counter() < t_end:
            step()
            n_pre += 1
            if n_pre % 8 == 0:
                torch.cuda.synchronize()   # keep the host within a few steps of the device
    for _ in range(warmup):
        step()
    res = {"T": T, "H": H, "D": D, "n_useful": n_useful, "segments": int(len(b.prefix)), "batch": b,
           "prewarm_steps": n_pre}
    res["ms"] = timed(step, steps)
    if fwd_split:
        def fwd_nograd():
            with torch.no_grad():
                fwd()
        res["fwd_calls"] = max(50, steps // 2)
        res["fwd_ms"] = timed(fwd_nograd, res["fwd_calls"])
        res["host_us"] = _host_us(b, q, k, v, seq)
    if timed_kernels:
        timer = _capi.Timer()
        timer.read()
        with timer:
            res["ms_timed"] = timed(step, steps)
        res["kernels"] = timer.read()
        timer.close()
    return res


def _hbm_bytes(T, H, D):
    """Algorithmic HBM bytes of one fwd+bwd step (bf16): forward reads Q, K, V and writes
    O (4 T H D 2) plus the LSE (4 T H); backward reads Q, K, V, O, dO and writes dQ, dK,
    dV (8 T H D 2) plus the LSE read and delta's write and read (12 T H)."""
    return 12 * T * H * D * 2 + 16 * T * H


def _host_us(b, q, k, v, seq, n=200):
    """Host time per forward and per backward op call (the ctypes dispatch, argument
    packing and output allocation), from a loop of n calls with no synchronization
    inside it: perf_counter around the loop, divided by n. The GPU work they launch is
    drained afterwards, outside the measurement."""
    import torch
    from prefixlm import op
    sc = 1.0 / (q.shape[-1] ** 0.5)
    vals = list(b.seq_info.values())
    plan, dsb = seq.get("plan"), seq.get("plan_ds_blocks")
    out, lse, lo, qa = op.varlen_fwd(b.q, b.k, b.v, False, *vals, sc, plan)
    torch.cuda.synchronize()
    res = {}
    for name, fn in (("fwd", lambda: op.varlen_fwd(b.q, b.k, b.v, False, *vals, sc, plan)),
                     ("bwd", lambda: op.varlen_bwd(b.q, b.k, b.v, False, b.dout, out, lse, lo, qa, *vals, sc,
                                                   plan, dsb))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        res[name] = round((time.perf_counter() - t0) / n * 1e6, 1)
        torch.cuda.synchronize()
    return res


def _case_summary(r):
    D, H, n = r["D"], r["H"], r["n_useful"]
    f = 14 * D * H * n
    out = {"tflops": round(f / (r["ms"] * 1e-3) / 1e12, 2), "pct_of_peak": round(100 * f / (r["ms"] * 1e-3) / 1e12
                                                                                    / PEAK_TFLOPS, 2),
           "ms_per_step": round(r["ms"], 4), "tokens": r["T"], "heads": H, "segments": r["segments"],
           "useful_tflop_per_step": round(f / 1e12, 4),
           "hbm_floor_ms": round(_hbm_bytes(r["T"], H, D) / (HBM_GBPS * 1e9) * 1e3, 4),
           "mfma_floor_ms": round(f / (PEAK_TFLOPS * 1e12) * 1e3, 4)}
    if "kernels" in r:
        out["kernel_avg_ms"] = {name: round(t / c, 4) for name, (t, c) in r["kernels"].items() if c}
    return out


if __name__ == "__main__":
    main()
