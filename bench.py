#!/usr/bin/env python3
"""Benchmark of the optimized pre-LN transformer forward on one MI355X.

Metric: p50 forward latency (us) per config, and fp16 MFMA TFLOP/s as a fraction of
the MI355X dense fp16 peak.  A "step" is one forward call ``opt(x, mask)`` of the headline
workload (default C5: 12 layers, D1024, H16, F4096, B2, S4096, causal) on resident fp16 inputs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C5] [--configs all|none|C1,..]

Prints ONE JSON line.  Per the reference harness (benchmarks/torch_transformer_benchmark.py:477-583)
every call is bracketed by HIP events on the current stream, the optimized and eager-fp16 models
alternate rounds, p50/p90 use the linearly interpolated percentile (:427-439) and
tokens/s = B*S / p50.  The K timed steps are also bracketed by a device synchronisation on both
sides, which gives ``ms_per_step``.  Inside the same run each kernel of one layer is timed in
isolation (HIP events on the stream it is launched on) to give the roofline of the dominant
kernel, and the CPU fp32 oracle is timed on a bounded sample on the host cores.

    python bench.py --mode cases

times the reference's own 14-case shape table (optimized_transformer.py:22-42) against eager fp16
instead and prints that as its one JSON line.
"""

from __future__ import annotations

import argparse
import copy
import json
import math
import os
import statistics
import sys
import time

import torch

from tttj_2026_amd import PLAN_LAYERWISE, _lib, make_optimized_transformer, ops, roofline
from tttj_2026_amd.configs import (REFERENCE_CASES, SEED, WORKLOADS, WORKLOAD_ORDER, build_model,
                                   make_inputs, reference_case_config, workload_inputs)

METRIC = "p50 fwd latency (us) per config; fp16 MFMA TFLOP/s as % of MI355X peak"
PEAK_TFLOPS = roofline.MI355X_FP16_DENSE_TFLOPS
PEAK_GBPS = roofline.MI355X_HBM_GBPS


def percentile(values, q):
    v = sorted(values)
    if len(v) == 1:
        return v[0]
    pos = (len(v) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    return v[lo] if lo == hi else v[lo] * (hi - pos) + v[hi] * (pos - lo)


def time_calls(fn, iters):
    """Per-call HIP-event times (ms) of ``fn`` on the current stream."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    torch.cuda.synchronize()
    for i in range(iters):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def loop_time(fn, iters):
    """Average ms per call of ``fn`` over ``iters`` back-to-back calls (HIP events)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def lengths_of(mask, cfg):
    if mask is None:
        return None
    return [int(v) for v in mask.sum(dim=1).tolist()]


def bench_workload(name, steps, warmup, rounds, eager, dev):
    x16, mask = workload_inputs(name)
    return bench_model(WORKLOADS[name].config, x16, mask, steps, warmup, rounds, eager, dev)


def bench_model(cfg, x16, mask, steps, warmup, rounds, eager, dev, xd=None):
    """Alternating rounds of optimized and eager fp16 forwards, per-call HIP-event times."""
    model = build_model(cfg).half().to(dev).eval()
    opt = make_optimized_transformer(copy.deepcopy(model))
    if xd is None:
        xd = x16.to(dev)
    md = None if mask is None else mask.to(dev)
    with torch.inference_mode():
        for _ in range(warmup):
            opt(xd, md)
        if eager:
            for _ in range(max(2, warmup // 4)):
                model(xd, md)
        torch.cuda.synchronize()
        opt_s, eager_s = [], []
        per = -(-steps // rounds)  # every round the same count, steps in all (at least)
        for r in range(rounds):
            order = (0, 1) if r % 2 == 0 else (1, 0)
            for which in order:
                if which == 0:
                    opt_s += time_calls(lambda: opt(xd, md), per)
                elif eager:
                    eager_s += time_calls(lambda: model(xd, md), per)
    p50 = statistics.median(opt_s)
    lens = lengths_of(mask, cfg)
    useful = roofline.forward_flops(cfg, lens)
    dense = roofline.forward_flops(cfg)
    out = {
        "p50_us": p50 * 1e3,
        "p90_us": percentile(opt_s, 0.9) * 1e3,
        "tokens_per_s": cfg.batch_size * cfg.seq_len / (p50 * 1e-3),
        "useful_gflop": useful / 1e9,
        "dense_gflop": dense / 1e9,
        "useful_tflops": useful / (p50 * 1e-3) / 1e12,
        "mfma_frac_useful": useful / (p50 * 1e-3) / 1e12 / PEAK_TFLOPS,
        "samples": len(opt_s),
    }
    if eager_s:
        e50 = statistics.median(eager_s)
        out.update(eager_p50_us=e50 * 1e3, eager_p90_us=percentile(eager_s, 0.9) * 1e3,
                   speedup_vs_eager=e50 / p50)
    return out, (model, opt, xd, md, x16, mask)


def kernel_breakdown(name, dev, iters=20):
    """Time each kernel of one layer in isolation (HIP events on the launch stream), on the data
    the forward itself runs them on: one forward of the workload leaves its last layer's Q / K /
    V^T (Q pre-multiplied by the softmax factor, the form its attention launches read), LN2 output
    and GELU activations in the workspace, and the GEMMs use that layer's packed weights.  The
    attention is the forward's variant (tt_attention_fwd_prescaled).  For masked workloads the
    forward packs the valid tokens; these isolated GEMMs run all B*S rows (an upper bound)."""
    cfg = WORKLOADS[name].config
    B, S, D, H, F, L = (cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                        cfg.num_layers)
    T, hd, Sp = B * S, D // H, (S + 63) // 64 * 64
    x16, mask = workload_inputs(name)
    model = build_model(cfg).half().to(dev).eval()
    opt = make_optimized_transformer(copy.deepcopy(model), plan=PLAN_LAYERWISE)
    xd = x16.to(dev)
    md = None if mask is None else mask.to(dev)
    with torch.inference_mode():
        opt(xd, md)
    torch.cuda.synchronize()
    ws = opt.last_workspace
    oq, _, oh = _lib.stage_offsets(B, S, D, H, F, L, PLAN_LAYERWISE)
    half = lambda off, n: ws[off:off + 2 * n].view(torch.float16)
    plane = T * D
    qkv = half(oq, 2 * plane + B * D * Sp)
    q, k, vt = (qkv[:plane].view(B, H, S, hd), qkv[plane:2 * plane].view(B, H, S, hd),
                qkv[2 * plane:].view(B, H, hd, Sp))
    xa = half(0, plane).view(T, D).clone()                     # residual stream
    xn = half((T * D * 2 + 255) // 256 * 256, plane).view(T, D).clone()   # LN2 output
    hmid = half(oh, T * F).view(T, F).clone()                  # GELU activations
    offs, stride, final_off, _ = _lib.weight_layout(D, F, L)
    wl = opt.packed_weights[(L - 1) * stride:]
    seg = lambda i, n: wl[offs[i]:offs[i] + n]
    lnw, lnb = seg(6, D), seg(7, D)
    wqkv, bqkv = seg(2, 3 * D * D).view(3 * D, D), seg(3, 3 * D)
    wo, bo = seg(4, D * D).view(D, D), seg(5, D)
    w1, b1 = seg(8, F * D).view(F, D), seg(9, F)
    w2, b2 = seg(10, D * F).view(D, F), seg(11, D)
    ctx = ops.attention(q, k, vt, md, cfg.causal, prescaled=True).reshape(T, D)
    resid = xa.clone()
    lens = lengths_of(mask, cfg)
    lf = roofline.layer_flops(cfg, lens)
    # The short launches (LayerNorm, attention) are timed through the C ABI with preallocated
    # outputs (and the mask summary computed once): the Python wrappers' per-call overhead would
    # otherwise leave the GPU idle between back-to-back launches.
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    y_ln = torch.empty_like(xa)
    ln_args = (xa.data_ptr(), lnw.data_ptr(), lnb.data_ptr(), None, y_ln.data_ptr(), T, D, 1e-5,
               stream)
    _lib.check(lib.tt_layernorm_fwd(*ln_args), "tt_layernorm_fwd")
    info = None if md is None else ops.mask_info(md, B, S, dev)
    ctx_out = torch.empty(B, S, D, dtype=torch.float16, device=dev)
    att_args = (q.data_ptr(), k.data_ptr(), vt.data_ptr(), None if md is None else md.data_ptr(),
                None if info is None else info.data_ptr(), ctx_out.data_ptr(), B, S, H, hd,
                int(cfg.causal), stream)
    _lib.check(lib.tt_attention_fwd_prescaled(*att_args), "tt_attention_fwd_prescaled")
    kernels = {
        "layernorm": (lambda: lib.tt_layernorm_fwd(*ln_args), 2, "hbm", roofline.layernorm_bytes(T, D)),
        "gemm_qkv": (lambda: ops.qkv_projection(xn.reshape(B, S, D), wqkv, bqkv, H), 1, "mfma",
                     2 * T * 3 * D * D),
        "attention": (lambda: lib.tt_attention_fwd_prescaled(*att_args), 1, "mfma",
                      lf["attention"]),
        "gemm_out": (lambda: ops.linear(ctx, wo, bo, "resid_masked", residual=resid, valid=md,
                                        out=resid), 1, "mfma", 2 * T * D * D),
        "gemm_ffn_in": (lambda: ops.linear(xn, w1, b1, "gelu"), 1, "mfma", 2 * T * D * F),
        "gemm_ffn_out": (lambda: ops.linear(hmid, w2, b2, "masked_resid", residual=resid,
                                            valid=md, out=resid), 1, "mfma", 2 * T * F * D),
    }
    res = {}
    for kname, (fn, per_layer, bound, work) in kernels.items():
        for _ in range(3):
            fn()
        # average over back-to-back launches between one pair of HIP events on the launch stream
        # (per-call event pairs would also count the host's launch latency as GPU time); the
        # median of 3 such loops
        t = statistics.median(loop_time(fn, iters) for _ in range(3))
        entry = {"avg_ms": t, "per_layer": per_layer, "bound": bound,
                 "ms_per_forward": t * per_layer * cfg.num_layers}
        if bound == "mfma":
            entry["achieved_tflops"] = work / (t * 1e-3) / 1e12
            entry["frac"] = entry["achieved_tflops"] / PEAK_TFLOPS
            entry["flops"] = work
        else:
            entry["achieved_gbps"] = work / (t * 1e-3) / 1e9
            entry["frac"] = entry["achieved_gbps"] / PEAK_GBPS
            entry["bytes"] = work
        res[kname] = entry
    return res


def library_gemms(name, dev, iters=20):
    """Each projection of one layer of ``name`` three ways on the same operands (the forward's
    residual stream and GELU activations, their LayerNorm with the last layer's norm2, the last
    layer's weights): this build's kernel
    with the forward's fused epilogue, this build's kernel with a bias-only epilogue, and the
    vendor library through torch (``F.linear``: hipBLASLt, bias fused), alone and followed by the
    unfused epilogue ops that would complete it (GELU, residual add).  Average per launch (us)."""
    import torch.nn.functional as Fn
    cfg = WORKLOADS[name].config
    B, S, D, H, F, L = (cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                        cfg.num_layers)
    T = B * S
    x16, mask = workload_inputs(name)
    model = build_model(cfg).half().to(dev).eval()
    opt = make_optimized_transformer(copy.deepcopy(model), plan=PLAN_LAYERWISE)
    xd = x16.to(dev)
    md = None if mask is None else mask.to(dev)
    with torch.inference_mode():
        opt(xd, md)
    torch.cuda.synchronize()
    ws = opt.last_workspace
    _, _, oh = _lib.stage_offsets(B, S, D, H, F, L, PLAN_LAYERWISE)
    half = lambda off, n: ws[off:off + 2 * n].view(torch.float16)
    xa = half(0, T * D).view(T, D).clone()  # the residual stream leads the workspace
    hmid = half(oh, T * F).view(T, F).clone()
    offs, stride, _, _ = _lib.weight_layout(D, F, L)
    wl = opt.packed_weights[(L - 1) * stride:]
    seg = lambda i, n: wl[offs[i]:offs[i] + n]
    xn = ops.layernorm(xa, seg(6, D), seg(7, D))  # an LN2 output of the forward's magnitude
    wqkv, bqkv = seg(2, 3 * D * D).view(3 * D, D), seg(3, 3 * D)
    wo, bo = seg(4, D * D).view(D, D), seg(5, D)
    w1, b1 = seg(8, F * D).view(F, D), seg(9, F)
    w2, b2 = seg(10, D * F).view(D, F), seg(11, D)
    ctx = xn.clone()  # an activation of the context's shape and magnitude
    resid = xa.clone()
    gemms = {
        "qkv": (lambda: ops.qkv_projection(xn.reshape(B, S, D), wqkv, bqkv, H),
                lambda: ops.linear(xn, wqkv, bqkv, "bias"),
                lambda: Fn.linear(xn, wqkv, bqkv), None, 2 * T * 3 * D * D),
        "out_proj": (lambda: ops.linear(ctx, wo, bo, "resid_masked", residual=resid, valid=md,
                                        out=resid),
                     lambda: ops.linear(ctx, wo, bo, "bias"),
                     lambda: Fn.linear(ctx, wo, bo), lambda y: y.add_(xa), 2 * T * D * D),
        "ffn_in": (lambda: ops.linear(xn, w1, b1, "gelu"), lambda: ops.linear(xn, w1, b1, "bias"),
                   lambda: Fn.linear(xn, w1, b1), lambda y: Fn.gelu(y), 2 * T * D * F),
        "ffn_out": (lambda: ops.linear(hmid, w2, b2, "masked_resid", residual=resid, valid=md,
                                       out=resid),
                    lambda: ops.linear(hmid, w2, b2, "bias"),
                    lambda: Fn.linear(hmid, w2, b2), lambda y: y.add_(xa), 2 * T * F * D),
    }
    res = {}
    with torch.inference_mode():
        for gname, (fused, bias, lib_fn, lib_epi, flops) in gemms.items():
            runs = {"ours_fused": fused, "ours_bias": bias, "library_bias": lib_fn}
            if lib_epi is not None:
                runs["library_plus_epilogue_ops"] = lambda f=lib_fn, g=lib_epi: g(f())
            entry = {"flops": flops}
            for tag, fn in runs.items():
                for _ in range(3):
                    fn()
                t = statistics.median(loop_time(fn, iters) for _ in range(3))
                entry[tag + "_us"] = t * 1e3
                entry[tag + "_frac"] = flops / (t * 1e-3) / 1e12 / PEAK_TFLOPS
            res[gname] = entry
    return res


COPY_ELEMS = 64 * 1024 * 1024  # fp16 elements: 128 MiB read + 128 MiB written per copy


def copy_calibration(dev, reps=3):
    """A plain device copy of known size; its FETCH_SIZE / WRITE_SIZE counters calibrate the
    counters read for the kernels (bytes per dispatch = 128 MiB each way)."""
    a = torch.ones(COPY_ELEMS, dtype=torch.float16, device=dev)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()


def load_traffic(name, kernel):
    """HBM bytes per launch of ``kernel`` at ``name`` from the committed rocprofv3 counter
    summary (profiles/traffic.json), or None when no counter run covers it."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
        return table[name][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError, TypeError):
        return None


# CPU fp32 repeats per workload (after a one-layer warm-up call), as the benchmark plan asks.
CPU_REPEATS = {"C1": 20, "C2": 20, "C3": 5, "C4": 3, "C5": 3}


def host_info():
    """Cores the CPU path may use on this host, and how that was decided."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = os.environ.get("OMP_NUM_THREADS")
    cores = affinity
    if omp and omp.isdigit() and int(omp) > 0:
        cores = min(cores, int(omp))  # the lease's CPU share (16 per GPU on the MI355X boxes)
    info = {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "omp_num_threads": omp, "cores": max(1, cores)}
    try:
        with open("/proc/cpuinfo") as f:
            text = f.read()
        info["cpu_model"] = next(l.split(":", 1)[1].strip() for l in text.splitlines()
                                 if l.startswith("model name"))
        phys = {(l1, l2) for l1, l2 in zip(
            [l.split(":", 1)[1].strip() for l in text.splitlines() if l.startswith("physical id")],
            [l.split(":", 1)[1].strip() for l in text.splitlines() if l.startswith("core id")])}
        info["physical_cores_host"] = len(phys) or None
    except Exception:
        pass
    return info


def cpu_baseline(name, gpu_out=None, reps=None):
    """Time the fp32 CPU oracle (this repo's restatement of BaselineTransformer) on host cores:
    one warm-up call of the first layer, then ``reps`` full forwards (median; p90 too)."""
    from oracle import transformer_oracle as O

    info = host_info()
    cores = info["cores"]
    torch.set_num_threads(cores)
    w = WORKLOADS[name]
    cfg = w.config
    model = build_model(cfg)
    params = O.params_fp32(copy.deepcopy(model).half())
    x16, mask = workload_inputs(name)
    x = x16.float()
    reps = reps or CPU_REPEATS.get(name, 3)
    first = {k: v for k, v in params.items()
             if not k.startswith("layers.") or int(k.split(".")[1]) < 1}
    O.forward(first, x, mask, cfg.num_heads, cfg.causal)  # warm-up (threads, allocator)
    times, y = [], None
    for _ in range(reps):
        t0 = time.perf_counter_ns()
        y = O.forward(params, x, mask, cfg.num_heads, cfg.causal)
        times.append((time.perf_counter_ns() - t0) / 1e3)
    result = {"unit": "us", "cores": cores, "kind": "port", "value": statistics.median(times),
              "p90_us": percentile(times, 0.9), "repeats": reps,
              "sample": f"{reps} full forward(s) of {name} after a one-layer warm-up, median",
              "torch_threads": torch.get_num_threads(),
              "tokens_per_s": cfg.batch_size * cfg.seq_len / (statistics.median(times) * 1e-6)}
    result.update({k: v for k, v in info.items() if k != "cores"})
    if gpu_out is not None:
        d = (gpu_out.float().cpu() - y).abs()
        result["gpu_vs_oracle"] = {"max_abs": float(d.max()), "mean_abs": float(d.mean())}
    return result


def bench_reference_cases(dev, rounds, eager):
    """The reference's own 14-case table (optimized_transformer.py:22-42; causal, F = D, no mask):
    optimized vs eager fp16 p50 per case.  Case 14 (S = 100000) has no eager number: its score
    tensor alone would be B*H*S^2 fp16 elements (10 PB)."""
    out = {}
    for case in sorted(REFERENCE_CASES):
        cfg = reference_case_config(case)
        heavy = cfg.batch_size * cfg.seq_len >= 1_000_000
        if case == 14:   # inputs made on the GPU (3.2M x 1024): host generation would take minutes
            g = torch.Generator(device=dev).manual_seed(SEED + 100 + case)
            xd = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g,
                             device=dev).half()
            x16 = None
        else:
            x16, _ = make_inputs(cfg, False, SEED + 100 + case)
            xd = None
        res, _ = bench_model(cfg, x16, None, 3 if case == 14 else (10 if heavy else 50),
                             1 if case == 14 else (3 if heavy else 20), 1 if heavy else rounds,
                             eager and case != 14, dev, xd=xd)
        res["shape_b_s_d_h"] = list(REFERENCE_CASES[case])
        res["layers"] = cfg.num_layers
        out[str(case)] = res
        print(f"[cases] {case} {REFERENCE_CASES[case]} p50 {res['p50_us']:.1f} us"
              + (f" eager {res['eager_p50_us']:.1f} us" if "eager_p50_us" in res else ""),
              file=sys.stderr, flush=True)
    sp = [v["speedup_vs_eager"] for v in out.values() if "speedup_vs_eager" in v]
    return {"mode": "reference_cases", "cases": out, "n_with_eager": len(sp),
            "geomean_speedup_vs_eager": math.exp(sum(map(math.log, sp)) / len(sp)) if sp else None,
            "gpu": torch.cuda.get_device_name(dev)}


def forward_runs(name, dev, steps, warmup):
    """The workload's own forward (the plan its shape resolves to), `steps` times after `warmup`:
    for rocprofv3 counter runs over exactly the kernels a forward of this workload launches."""
    cfg = WORKLOADS[name].config
    x16, mask = workload_inputs(name)
    opt = make_optimized_transformer(build_model(cfg).half().to(dev).eval())
    xd = x16.to(dev)
    md = None if mask is None else mask.to(dev)
    plan = _lib.resolve_plan(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                             opt.plan)
    with torch.inference_mode():
        for _ in range(warmup):
            opt(xd, md)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            opt(xd, md)
        torch.cuda.synchronize()
    return {"workload": name, "plan": plan, "steps": steps,
            "ms_per_forward": (time.perf_counter() - t0) * 1e3 / max(steps, 1),
            "packed_rows": bool(md is not None and _lib.forward_packs_rows(
                cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim, plan))}


MEGA_KINDS = ("qkv", "attention", "out_proj", "ffn_in", "ffn_out")


def megakernel_trace_summary(name, dev, reps=20):
    """Per-task trace of the persistent megakernel (forward_traced) on the workload's shape, per
    layer and task kind (stage): the task count, the median run time (dependencies met -> end)
    and, relative to the launch's first task start, when the stage's first and median task had
    its dependencies met and when its last task ended (the critical path); also how busy the
    workgroups were.  Medians over `reps` launches; times in us (the trace clock is 100 MHz).
    Task numbering per layer: QKV (row blocks x 3D/64 tiles), attention (B x H x query blocks of
    128), out_proj (row blocks x D/64), ffn_in (row blocks x F/64), ffn_out (row blocks x D/64 x K
    splits), then one final LayerNorm task per row block (csrc/megakernel.hip,
    megakernel_tasks)."""
    cfg = WORKLOADS[name].config
    x16, mask = workload_inputs(name)
    opt = make_optimized_transformer(build_model(cfg).half().to(dev).eval())
    xd = x16.to(dev)
    md = None if mask is None else mask.to(dev)
    B, S, D, H, F, L = (cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                        cfg.num_layers)
    nrb = B * -(-S // 64)
    nqb = -(-S // 128)
    with torch.inference_mode():
        traces = [opt.forward_traced(xd, md)[1].tolist() for _ in range(reps)]
    ntask = len(traces[0])
    per_layer = (ntask - nrb) // L
    counts = [nrb * 3 * D // 64, B * H * nqb, nrb * D // 64, nrb * F // 64]
    counts.append(per_layer - sum(counts))
    kind_of = []
    for k, c in enumerate(counts):
        kind_of += [k] * c

    def stage(task):
        if task >= L * per_layer:
            return (L, "final_norm")
        return (task // per_layer, MEGA_KINDS[kind_of[task % per_layer]])

    spans, busy = [], []
    acc = {}
    for t in traces:
        t0 = min(r[1] for r in t)
        t1 = max(r[3] for r in t)
        spans.append((t1 - t0) / 100.0)
        wgs = len({r[0] >> 32 for r in t})
        busy.append(sum(r[3] - r[1] for r in t) / (wgs * (t1 - t0)))
        per = {}
        for task, r in enumerate(t):
            per.setdefault(stage(task), []).append(r)
        for key, rs in per.items():
            ready = sorted((r[2] - t0) / 100.0 for r in rs)
            a = acc.setdefault(key, {"run": [], "first_ready": [], "ready": [], "last_end": []})
            a["run"] += [(r[3] - r[2]) / 100.0 for r in rs]
            a["first_ready"].append(ready[0])
            a["ready"].append(statistics.median(ready))
            a["last_end"].append(max((r[3] - t0) / 100.0 for r in rs))
    rows = []
    for (layer, kind) in sorted(acc, key=lambda k: (k[0], MEGA_KINDS.index(k[1])
                                                     if k[1] in MEGA_KINDS else 9)):
        a = acc[(layer, kind)]
        rows.append({"layer": layer if kind != "final_norm" else -1, "kind": kind,
                     "tasks": len(a["run"]) // reps,
                     "run_us_p50": statistics.median(a["run"]),
                     "first_ready_us": statistics.median(a["first_ready"]),
                     "ready_us_p50": statistics.median(a["ready"]),
                     "last_end_us": statistics.median(a["last_end"])})
    return {"workload": name, "tasks": ntask,
            "workgroups": len({r[0] >> 32 for r in traces[-1]}),
            "span_us_p50": statistics.median(spans), "busy_frac_p50": statistics.median(busy),
            "per_layer_kind": rows}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="C5", choices=WORKLOAD_ORDER)
    ap.add_argument("--configs", default="all", help="all | none | comma list of C1..C5")
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-eager", action="store_true")
    ap.add_argument("--mode", default="full",
                    choices=("full", "kernels", "forward", "trace", "cases", "library"),
                    help="kernels: only run each kernel of one layer (and a copy of known size) "
                         "a few times, for rocprofv3 counter runs; forward: only run the "
                         "workload's own forward --steps times; trace: per-task summary of the "
                         "megakernel's trace on the workload's shape; cases: time the "
                         "reference's own 14-case shape table against eager fp16 (one JSON line); "
                         "library: each projection of one layer against the vendor library "
                         "(F.linear, hipBLASLt) on the same operands")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the forward would shard by sequence with zero collectives; not built)",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    name = args.workload
    cfg = WORKLOADS[name].config
    if args.mode == "cases":
        print(json.dumps(bench_reference_cases(dev, args.rounds, not args.no_eager)))
        return 0
    if args.mode == "forward":
        copy_calibration(dev)
        print(json.dumps(forward_runs(name, dev, args.steps, args.warmup)))
        return 0
    if args.mode == "trace":
        print(json.dumps(megakernel_trace_summary(name, dev)))
        return 0
    if args.mode == "library":
        copy_calibration(dev)
        print(json.dumps({"workload": name, "gemms": library_gemms(name, dev, iters=args.steps)}))
        return 0
    if args.mode == "kernels":
        copy_calibration(dev)
        res = kernel_breakdown(name, dev, iters=args.steps)
        print(json.dumps({"workload": name, "kernels": res}))
        return 0

    # the p50 / p90 rest on at least 30 samples of each provider, whatever --steps is
    head, (model, opt, xd, md, x16, mask) = bench_workload(
        name, max(args.steps, 30), max(args.warmup, 5), args.rounds, not args.no_eager, dev)
    # the K timed steps, bracketed by synchronisation
    with torch.inference_mode():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            y = opt(xd, md)
        torch.cuda.synchronize()
        ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    print(f"[bench] {name} p50 {head['p50_us']:.1f} us", file=sys.stderr, flush=True)

    kernels = kernel_breakdown(name, dev)
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["ms_per_forward"])
    if dom["bound"] == "mfma":
        rl = {"kernel": dom_name, "bound": "mfma", "achieved": dom["achieved_tflops"],
              "peak": PEAK_TFLOPS, "unit": "TFLOP/s", "frac": dom["frac"],
              "traffic": load_traffic(name, dom_name),
              "work_per_launch": dom["flops"], "avg_launch_ms": dom["avg_ms"]}
    else:
        rl = {"kernel": dom_name, "bound": "hbm", "achieved": dom["achieved_gbps"],
              "peak": PEAK_GBPS, "unit": "GB/s", "frac": dom["frac"],
              "traffic": load_traffic(name, dom_name),
              "work_per_launch": dom["bytes"], "avg_launch_ms": dom["avg_ms"]}

    per_config = {}
    wanted = [] if args.configs == "none" else (
        list(WORKLOAD_ORDER) if args.configs == "all" else args.configs.split(","))
    for other in wanted:
        if other == name:
            per_config[other] = head
            continue
        per_config[other], _ = bench_workload(other, 100 if other in ("C1", "C2", "C3") else 30,
                                              20, args.rounds, not args.no_eager, dev)
        print(f"[bench] {other} p50 {per_config[other]['p50_us']:.1f} us", file=sys.stderr,
              flush=True)
    speedups = [v["speedup_vs_eager"] for v in per_config.values() if "speedup_vs_eager" in v]

    cpu = None
    if not args.no_cpu:
        # every benchmarked workload's CPU fp32 path, same run, same host; the headline's is
        # also `cpu_baseline`
        for other in [name] + [c for c in per_config if c != name]:
            res = cpu_baseline(other, gpu_out=y if other == name else None)
            print(f"[bench] {other} cpu fp32 p50 {res['value'] / 1e3:.1f} ms on {res['cores']} "
                  "cores", file=sys.stderr, flush=True)
            if other == name:
                cpu = res
            if other in per_config:
                per_config[other]["cpu_fp32"] = res
                per_config[other]["speedup_vs_cpu"] = res["value"] / per_config[other]["p50_us"]

    line = {
        "metric": METRIC,
        "value": head["p50_us"],
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded N(0,1) fp16 inputs, seeded default-init weights (no checkpoint)",
        "config": {"workload": name, "batch": cfg.batch_size, "seq_len": cfg.seq_len,
                   "d_model": cfg.d_model, "heads": cfg.num_heads, "ffn_dim": cfg.ffn_dim,
                   "layers": cfg.num_layers, "causal": cfg.causal,
                   "mask": "right-padded l~U{S/2..S}" if WORKLOADS[name].masked else "none",
                   "parallelism": "single-gpu"},
        "p90_us": head["p90_us"],
        "tokens_per_s": head["tokens_per_s"],
        "useful_tflops": head["useful_tflops"],
        "mfma_frac_useful": head["mfma_frac_useful"],
        "eager_fp16_p50_us": head.get("eager_p50_us"),
        "speedup_vs_eager": head.get("speedup_vs_eager"),
        "roofline": rl,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "per_config": per_config,
        "geomean_speedup_vs_eager": (math.exp(sum(map(math.log, speedups)) / len(speedups))
                                     if speedups else None),
        "gpu": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
