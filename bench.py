"""Benchmark Kiln's MI355X backend on BASELINE.json's metric (1 GPU).

    python bench.py [--steps K] [--warmup W] [--tokens T] [--quick]

Headline (the timed steps): one GPT-2-small block (pre-LN, d 768, 12 heads,
causal, fp32, random init N(0, 0.02), LN gamma 1 / beta 0, seeded input
[T, 768] ~ N(0, 1)) compiled by kiln.compile(device="cuda", autotune=True);
a step is one call as a user makes it (copy input in, one hipGraph replay of
the 11-launch plan, clone output out). `value` = ms per step, averaged over
exactly K steps between synchronisations, after W warm-up steps.

Also reported (outside the timed steps): block latency at 128/512/1024/2048
tokens with eager PyTorch beside it, the GEMM sweep in TFLOP/s, the fused
memory-bound ops in GB/s (hot = same buffers, as the reference times them;
cold = buffers rotated over > 512 MiB so the 256 MiB Infinity Cache cannot
hold them), the 12-layer stack, the roofline of the block's dominant kernel,
and the CPU baseline: the C oracle (float64, one thread) timed on this host
on one block at the headline size.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "kiln-compiler_amd"), ROOT, os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2516.6


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tokens", type=int, default=2048)
    p.add_argument("--quick", action="store_true", help="headline, roofline and CPU baseline only")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-autotune", action="store_true")
    return p.parse_args()


# -- timing helpers -----------------------------------------------------------------------

def events_ms(fn, iters):
    """Average ms of `fn` over `iters` back-to-back calls, HIP events on the
    current stream."""
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def graph_ms(fn, repeats=20, rounds=5):
    from kiln.hip.runtime import kernel_seconds

    return kernel_seconds(fn, repeats=repeats, rounds=rounds) * 1e3


def ms_per_call(fn, rounds=5, min_time=0.05):
    """Best-of-rounds wall ms per call measured with events (end to end)."""
    import torch

    for _ in range(3):
        fn()
    one = events_ms(fn, 1)
    calls = max(1, int(min_time * 1e3 / max(one, 1e-3)))
    return min(events_ms(fn, calls) for _ in range(rounds))


# -- workloads ------------------------------------------------------------------------------

def make_block(T, seed=0):
    import torch

    from models.transformer import Block, gpt2_init_

    torch.manual_seed(seed)
    model = gpt2_init_(Block(768, 12, T), seed=seed).eval().cuda()
    x = torch.randn(T, 768, generator=torch.Generator().manual_seed(seed + 1)).cuda()
    return model, x


def block_flops(T):
    return 14155776 * T + 3072 * T * T


def headline(args):
    import torch

    import kiln

    T = args.tokens
    model, x = make_block(T)
    t0 = time.perf_counter()
    compiled = kiln.compile(model, (x,), device="cuda", autotune=not args.no_autotune)
    log(f"compiled block T={T} in {time.perf_counter() - t0:.1f}s: {compiled.report.lowering['launches']} launches")
    with torch.no_grad():
        ref = model(x)
    out = compiled(x)
    err = (out - ref).abs().max().item()
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-5)
    for _ in range(args.warmup):
        compiled(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        compiled(x)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    return compiled, model, x, ms, err


def dominant_kernel_roofline(compiled, x):
    """Roofline of the block's longest launch: algorithmic bytes or flops per
    launch / its average duration (HIP events over back-to-back launches on
    the stream the kernel runs on)."""
    import torch

    from kiln.hip.runtime import current_stream_handle

    exe = compiled._exe
    prof = exe.profile(x)
    name, _ = max(prof, key=lambda p: p[1])
    idx = [l.name for l in exe.program.launches].index(name)
    launch = exe.program.launches[idx]
    inputs = exe._prepare((x,))
    outputs = [torch.empty(s, device=x.device) for s in exe.output_shapes]
    ins, outs = [t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs]
    fn = lambda: exe.plan.run_one(idx, ins, outs, current_stream_handle())
    for _ in range(5):
        fn()
    avg_ms = min(events_ms(fn, 200) for _ in range(3))
    if launch.flops:
        achieved = launch.flops / (avg_ms * 1e-3) / 1e12
        bound, peak, unit = "mfma", FP32_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved = launch.bytes / (avg_ms * 1e-3) / 1e9
        bound, peak, unit = "hbm", HBM_PEAK_GBS, "GB/s"
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": None,
            "kernel": name, "summary": launch.summary, "avg_us": round(avg_ms * 1e3, 2),
            "algorithmic": launch.flops or launch.bytes}, prof


def block_sweep(tokens, autotune):
    import torch

    import kiln

    out = {}
    for T in tokens:
        model, x = make_block(T)
        c = kiln.compile(model, (x,), device="cuda", autotune=autotune)
        with torch.no_grad():
            torch.testing.assert_close(c(x), model(x), rtol=1e-4, atol=1e-5)
            k_ms = ms_per_call(lambda: c(x))
            e_ms = ms_per_call(lambda: model(x))
            c._exe.replay_only()
            replay_ms = min(events_ms(c._exe.replay_only, 20) for _ in range(5))
        out[str(T)] = {"kiln_ms": round(k_ms, 4), "eager_ms": round(e_ms, 4), "replay_ms": round(replay_ms, 4),
                       "speedup": round(e_ms / k_ms, 3), "tflops": round(block_flops(T) / k_ms / 1e9, 2),
                       "arena_mib": round(c.report.arena_bytes / 2**20, 2)}
        log(f"block T={T}: kiln {k_ms:.4f} ms (replay {replay_ms:.4f}), eager {e_ms:.4f} ms")
    return out


def gemm_sweep(autotune):
    import torch

    import kiln
    from models.transformer import gpt2_init_

    shapes = [(2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768), (128, 768, 3072),
              (1, 3072, 768)]
    out = {}
    for m, n, k in shapes:
        torch.manual_seed(0)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=1).eval().cuda()
        x = torch.randn(m, k, device="cuda")
        c = kiln.compile(lin, (x,), device="cuda", autotune=autotune, cuda_graphs=False)
        with torch.no_grad():
            torch.testing.assert_close(c(x), lin(x), rtol=1e-4, atol=1e-5)
            outs = [torch.empty(m, n, device="cuda")]
            kms = graph_ms(lambda: c._exe.run_into([x], outs))
            ems = graph_ms(lambda: lin(x))
        flops = 2 * m * n * k
        out[f"{m}x{n}x{k}"] = {"kiln_tflops": round(flops / kms / 1e9, 2), "torch_tflops": round(flops / ems / 1e9, 2),
                               "kiln_us": round(kms * 1e3, 2)}
        log(f"gemm {m}x{n}x{k}: kiln {flops / kms / 1e9:.1f} TFLOP/s, torch {flops / ems / 1e9:.1f}")
    return out


def fused_ops():
    import torch
    import torch.nn.functional as F

    import kiln

    torch.manual_seed(0)
    bias = torch.randn(3072, device="cuda")
    ln = torch.nn.LayerNorm(768).eval().cuda()
    with torch.no_grad():
        ln.weight.copy_(1 + torch.randn(768) * 0.02)
        ln.bias.copy_(torch.randn(768) * 0.02)
    work = [
        ("bias_gelu_2048x3072", lambda t: F.gelu(t + bias, approximate="tanh"), (2048, 3072),
         (2 * 2048 * 3072 + 3072) * 4),
        ("layernorm_2048x768", ln, (2048, 768), (2 * 2048 * 768 + 2 * 768) * 4),
        ("softmax_12x512x512", lambda t: F.softmax(t * 0.125, -1), (12, 512, 512), 2 * 12 * 512 * 512 * 4),
    ]
    out = {}
    for name, fn, shape, nbytes in work:
        x = torch.randn(*shape, device="cuda")
        c = kiln.compile(fn, (x,), device="cuda", cuda_graphs=False)
        with torch.no_grad():
            torch.testing.assert_close(c(x), fn(x), rtol=1e-4, atol=1e-5)
        y = torch.empty(shape, device="cuda")
        hot = graph_ms(lambda: c._exe.run_into([x], [y]))
        # cold: rotate over enough buffers to exceed twice the 256 MiB Infinity Cache
        per = 2 * math.prod(shape) * 4
        n = max(4, math.ceil(640 * 2**20 / per))
        xs = [torch.randn(*shape, device="cuda") for _ in range(n)]
        ys = [torch.empty(shape, device="cuda") for _ in range(n)]
        state = {"i": 0}

        def step():
            i = state["i"] % n
            state["i"] += 1
            c._exe.run_into([xs[i]], [ys[i]])

        cold = graph_ms(step, repeats=n, rounds=3)
        with torch.no_grad():
            eager = graph_ms(lambda: fn(x))
        out[name] = {"kiln_hot_us": round(hot * 1e3, 2), "kiln_cold_us": round(cold * 1e3, 2),
                     "eager_hot_us": round(eager * 1e3, 2),
                     "hot_gbs": round(nbytes / hot / 1e6, 1), "cold_gbs": round(nbytes / cold / 1e6, 1),
                     "cold_hbm_frac": round(nbytes / cold / 1e6 / HBM_PEAK_GBS, 3), "bytes": nbytes}
        log(f"{name}: hot {hot * 1e3:.2f} us ({nbytes / hot / 1e6:.0f} GB/s), cold {cold * 1e3:.2f} us "
            f"({nbytes / cold / 1e6:.0f} GB/s), eager {eager * 1e3:.2f} us")
        del xs, ys
        torch.cuda.empty_cache()
    return out


def stack_bench(autotune):
    import torch

    import kiln
    from models.transformer import Stack, gpt2_init_

    out = {}
    for name, T in (("prefill_1024", 1024), ("decode_1", 1)):
        torch.manual_seed(0)
        model = gpt2_init_(Stack(12, 768, 12, T), seed=0).eval().cuda()
        x = torch.randn(T, 768, device="cuda")
        c = kiln.compile(model, (x,), device="cuda", autotune=autotune)
        with torch.no_grad():
            torch.testing.assert_close(c(x), model(x), rtol=1e-3, atol=1e-4)
            k_ms = ms_per_call(lambda: c(x))
            e_ms = ms_per_call(lambda: model(x))
        flops = 12 * block_flops(T)
        out[name] = {"kiln_ms": round(k_ms, 4), "eager_ms": round(e_ms, 4), "tflops": round(flops / k_ms / 1e9, 2),
                     "launches": c.report.lowering["launches"]}
        log(f"stack {name}: kiln {k_ms:.4f} ms, eager {e_ms:.4f} ms")
    return out


def cpu_baseline(T):
    """The C oracle (float64, single thread) on one block at the headline size."""
    import numpy as np
    import torch

    import oracle
    from models.transformer import Block, gpt2_init_

    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768, generator=torch.Generator().manual_seed(1)).numpy()
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    oracle.lib()
    t0 = time.perf_counter()
    oracle.block(x, params, 12)
    dt = time.perf_counter() - t0
    return {"value": round(dt * 1e3, 1), "unit": "ms", "cores": 1, "kind": "port",
            "sample": f"one full GPT-2 block forward at T={T} by oracle/kiln_oracle.c (float64, 1 thread)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        sys.exit("bench.py needs an MI355X (no ROCm GPU visible)")
    from kiln.hip import lib as kl

    torch.manual_seed(0)
    info = kl.device_info() if kl.load() else {}
    compiled, model, x, ms, err = headline(args)
    log(f"headline: block T={args.tokens}: {ms:.4f} ms/step over {args.steps} steps (max err {err:.2e})")
    roofline, prof = dominant_kernel_roofline(compiled, x)
    log("per-launch ms: " + ", ".join(f"{n}={t:.4f}" for n, t in prof))
    extra = {}
    if not args.quick:
        extra["block"] = block_sweep([128, 512, 1024, 2048], not args.no_autotune)
        extra["gemm"] = gemm_sweep(not args.no_autotune)
        extra["fused_ops"] = fused_ops()
        extra["stack"] = stack_bench(not args.no_autotune)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.tokens)
    line = {
        "metric": "GPT-2 block latency ms @128-2048 tok; GEMM TFLOP/s; fused-op GB/s (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (seeded N(0,1) input, random-init N(0,0.02) weights)",
        "config": {"workload": f"gpt2_small_block_T{args.tokens}", "tokens": args.tokens, "d_model": 768,
                   "heads": 12, "parallelism": "none (1 GPU)"},
        "roofline": roofline, "cpu_baseline": cpu,
        "device": info, "per_launch_ms": {n: round(t, 5) for n, t in prof}, **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
