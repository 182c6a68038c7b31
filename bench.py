"""Benchmark Kiln's MI355X backend on BASELINE.json's metric (1 GPU).

    python bench.py [--steps K] [--warmup W] [--tokens T] [--quick]

Headline (the timed steps): one GPT-2-small block (pre-LN, d 768, 12 heads,
causal, fp32, random init N(0, 0.02), LN gamma 1 / beta 0, seeded input
[T, 768] ~ N(0, 1)) compiled by kiln.compile(device="cuda", autotune=True);
a step is one call as a user makes it, with the input already in HBM: the
plan's launches run on the caller's tensors ("direct"), or the input is
copied into the static buffers, the captured hipGraph is replayed and the
output cloned ("graph"), whichever the executable's first call measured
faster (config.call_mode says which; the block sweep reports both paths at
every T). `value` = ms per step, averaged over exactly K steps between
synchronisations, after W warm-up steps.

Also reported (outside the timed steps, and run before them so the timed
steps see a GPU whose clocks are up): block latency at 128/512/1024/2048
tokens with eager PyTorch and torch.compile(mode="reduce-overhead") beside it
and the per-call memory of each, the GEMM sweep in TFLOP/s, the fused
memory-bound ops in GB/s (hot = same buffers, as the reference times them;
cold = buffers rotated over > 512 MiB so the 256 MiB Infinity Cache cannot
hold them), the 12-layer stack, the roofline of the block's dominant kernel,
and the CPU baseline: the C oracle (the port of the reference's algorithm,
float64, one thread) on the headline block, with eager PyTorch CPU fp32 on the
same block at one thread and at all the cores the process may use (best of
3, the reference's bench_block.py method) as separately labelled lines.
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
    p.add_argument("--steps", type=int, default=50)
    # 300 untimed calls (~0.1 s at T = 2048) bring the GPU's clocks up: after
    # 10 the first timed calls still run ~5% slower
    p.add_argument("--warmup", type=int, default=300)
    p.add_argument("--tokens", type=int, default=2048)
    p.add_argument("--quick", action="store_true", help="headline, roofline and CPU baseline only")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-autotune", action="store_true")
    p.add_argument("--no-inductor", action="store_true", help="skip the torch.compile column of the block sweep")
    p.add_argument("--counter-probe", metavar="JSON",
                   help="run only the dispatch sequence the rocprofv3 --pmc passes count (a copy of known size, "
                        "then every launch of the block plans, a bf16 GEMM and torch's GEMMs, the fused ops, the "
                        "12-layer decode and the bf16 block, each repeated) and write its map to JSON")
    p.add_argument("--traffic-report", nargs=3, metavar=("PROBE_JSON", "FETCH_DIR", "WRITE_DIR"),
                   help="turn the FETCH_SIZE and WRITE_SIZE counter passes over --counter-probe into the "
                        "per-launch HBM traffic summary (no GPU needed); --tokens picks the block")
    p.add_argument("--traffic-groups", metavar="PREFIX",
                   help="with --traffic-report: the probe groups whose label starts with PREFIX (e.g. c2_, "
                        "decode12, bf16_T2048) instead of one block's launches")
    p.add_argument("--probes", action="store_true",
                   help="run only the library's measurement probes and print their summary: the MFMA / VALU "
                        "issue probe, and the attention kernel's per-workgroup timeline on the T = 2048 block "
                        "shape (12 heads; also 4 heads, one workgroup per CU)")
    p.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                   help="summarise a rocprofv3 --kernel-trace CSV of a bench.py run: kiln kernels per kernel and "
                        "grid, median and minimum duration (no GPU needed)")
    p.add_argument("--counter-report", nargs="+", metavar="PROBE_JSON DIR",
                   help="turn SQ counter passes over --counter-probe into the per-launch MFMA utilisation, "
                        "wait and LDS summary (no GPU needed)")
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


def peak_mib(fn, *xs):
    """MiB allocated by one call beyond what was allocated before it (the
    reference's per-call peak, benchmarks/bench_gpu.py:91-102)."""
    import torch

    with torch.no_grad():
        fn(*xs)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        fn(*xs)
        torch.cuda.synchronize()
    return (torch.cuda.max_memory_allocated() - base) / 2**20


def inductor_ms(fn, x, mode):
    """ms per call of torch.compile(fn, mode=mode) (Inductor's Triton kernels;
    "reduce-overhead" replays them as a graph), or None when it cannot run."""
    import torch

    try:
        compiled = torch.compile(fn, mode=mode)
        with torch.no_grad():
            torch.testing.assert_close(compiled(x), fn(x), rtol=1e-3, atol=1e-4)
            return ms_per_call(lambda: compiled(x))
    except Exception as err:  # noqa: BLE001 - a missing or failing compiler only drops the column
        log(f"  torch.compile unavailable: {str(err).splitlines()[0][:120]}")
        return None


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


def prepare_headline(args):
    """Compile the headline block and check it against eager PyTorch (done
    before the untimed sections, so nothing but the warm-up separates them
    from the timed steps)."""
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
    return compiled, model, x, err


def time_headline(args, compiled, x):
    """W untimed calls, then exactly K timed calls between synchronisations."""
    import torch

    for _ in range(args.warmup):
        compiled(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        compiled(x)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / args.steps


def dominant_kernel_roofline(compiled, x, T):
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
    traffic = committed_traffic(T, launch)
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic,
            "traffic_source": os.path.relpath(TRAFFIC_FILE.format(T=T), ROOT) if traffic else None,
            "kernel": name, "summary": launch.summary, "avg_us": round(avg_ms * 1e3, 2),
            "algorithmic": launch.flops or launch.bytes}, prof


# -- counters (rocprofv3 --pmc): HBM traffic, MFMA utilisation, waits, LDS --------------------

PROBE_REPS = 20
COPY_BYTES = 256 * 2**20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_block_T{T}.txt")
PROBE_TOKENS = (2048, 128)
PROBE_GEMM = (2048, 3072, 768)


def counter_probe(args):
    """The dispatch sequence the counter passes read: PROBE_REPS plain copies of
    COPY_BYTES (the calibration kernel: it reads and writes exactly COPY_BYTES),
    then groups, each a one-element fill (the group marker) followed by one
    launch PROBE_REPS times: every launch of the block plan at each of
    PROBE_TOKENS, the bf16-input GEMM of PROBE_GEMM (nn.Linear with bias),
    torch's own fp32 and bf16 products of the same shape (hipBLASLt) for
    comparison, the BASELINE fused ops (bias + GELU, LayerNorm, softmax), every
    launch of the 12-layer decode (one-row GEMVs) and of the bf16 block at
    T = 2048. A launch may issue several kernels (split-K issues two), so
    groups are cut at the markers. Writes the map from groups to launches as
    JSON."""
    import torch
    import torch.nn.functional as F

    import kiln
    from kiln.hip.runtime import current_stream_handle
    from models.transformer import gpt2_init_

    src = torch.empty(COPY_BYTES // 4, device="cuda").normal_()
    dst = torch.empty_like(src)
    marker = torch.empty(1, device="cuda")
    groups, runs = [], []

    def plan_groups(label, compiled, x):
        exe = compiled._exe
        inputs = exe._prepare((x,))
        outputs = [torch.empty(s, device=x.device) for s in exe.output_shapes]
        ins, outs = [t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs]
        exe.run_into(inputs, outputs)
        for i, l in enumerate(exe.program.launches):
            groups.append({"group": f"{label}/{l.name}", "name": l.name, "kernel": l.kernel, "summary": l.summary,
                           "flops": l.flops, "bytes": l.bytes})
            runs.append((lambda i=i, exe=exe, ins=ins, outs=outs, keep=(inputs, outputs):
                         exe.plan.run_one(i, ins, outs, current_stream_handle())))

    for T in PROBE_TOKENS:
        model, x = make_block(T)
        plan_groups(f"T{T}", kiln.compile(model, (x,), device="cuda", autotune=not args.no_autotune), x)
    m, n, k = PROBE_GEMM
    torch.manual_seed(0)
    lin = gpt2_init_(torch.nn.Linear(k, n), seed=1).eval().cuda()
    x = torch.randn(m, k, device="cuda")
    plan_groups(f"gemm_bf16_{m}x{n}x{k}", kiln.compile(lin, (x,), device="cuda", autotune=not args.no_autotune,
                                                      cuda_graphs=False, matmul_precision="bf16"), x)
    w, b = lin.weight.detach(), lin.bias.detach()
    xb, wb, bb = x.bfloat16(), w.bfloat16().contiguous(), b.bfloat16()
    flops = 2 * m * n * k
    for label, fn, nbytes in ((f"torch_fp32_{m}x{n}x{k}", lambda: F.linear(x, w, b), 4 * (m * k + k * n + n + m * n)),
                              (f"torch_bf16_{m}x{n}x{k}", lambda: F.linear(xb, wb, bb), 2 * (m * k + k * n + n + m * n))):
        groups.append({"group": label, "name": label, "kernel": "torch", "summary": f"F.linear {m}x{n}x{k}",
                       "flops": flops, "bytes": nbytes})
        runs.append(fn)
    # the BASELINE fused memory-bound ops (their launches' algorithmic bytes
    # are the table's: inputs and parameters read once, outputs written once)
    torch.manual_seed(0)
    bias = torch.randn(3072, device="cuda")
    ln = torch.nn.LayerNorm(768).eval().cuda()
    for label, fn, shape in (("c2_bias_gelu_2048x3072", lambda t: F.gelu(t + bias, approximate="tanh"), (2048, 3072)),
                             ("c2_layernorm_2048x768", ln, (2048, 768)),
                             ("c2_softmax_12x512x512", lambda t: F.softmax(t * 0.125, -1), (12, 512, 512))):
        xt = torch.randn(*shape, device="cuda")
        plan_groups(label, kiln.compile(fn, (xt,), device="cuda", cuda_graphs=False), xt)
    # the 12-layer decode: 49 one-row launches (GEMVs with their prologues)
    from models.transformer import Stack

    torch.manual_seed(0)
    stack = gpt2_init_(Stack(12, 768, 12, 1), seed=0).eval().cuda()
    x1 = torch.randn(1, 768, device="cuda")
    plan_groups("decode12", kiln.compile(stack, (x1,), device="cuda", autotune=not args.no_autotune,
                                         cuda_graphs=False), x1)
    # the bf16 block at T = 2048 (bf16 GEMMs, fp32 attention and rows)
    model, x = make_block(2048)
    plan_groups("bf16_T2048", kiln.compile(model, (x,), device="cuda", autotune=not args.no_autotune,
                                           matmul_precision="bf16"), x)
    torch.cuda.synchronize()
    with torch.no_grad():
        for _ in range(PROBE_REPS):
            dst.copy_(src)
        torch.cuda.synchronize()
        for i, run in enumerate(runs):
            marker.fill_(float(i))
            for _ in range(PROBE_REPS):
                run()
            torch.cuda.synchronize()
    info = {"reps": PROBE_REPS, "copy_bytes": COPY_BYTES, "marker": "FillFunctor", "groups": groups}
    with open(args.counter_probe, "w") as f:
        json.dump(info, f, indent=1)
    log(f"counter probe: copy x{PROBE_REPS}, then {len(groups)} marked launch groups x{PROBE_REPS}")


def _counter_rows(path):
    """Per-dispatch counter values from a rocprofv3 csv output tree, in
    dispatch order: [(kernel name, {counter: (sum, max) over instances})]."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {path}")
    per = {}
    for fn in files:
        with open(fn, newline="") as f:
            for row in csv.DictReader(f):
                key = int(row["Dispatch_Id"])
                name, vals = per.setdefault(key, (row["Kernel_Name"], {}))
                s, mx = vals.get(row["Counter_Name"], (0.0, 0.0))
                v = float(row["Counter_Value"])
                vals[row["Counter_Name"]] = (s + v, max(mx, v))
    return [per[k] for k in sorted(per)]


def _probe_groups(rows, probe):
    """Split the probe's dispatches: the copies right before the first marker,
    then one group per launch between markers. Returns (copies, groups): per
    repetition, {counter: (sum, max)} summed over the kernels of a launch."""
    reps, n = probe["reps"], len(probe["groups"])
    marks = [i for i, (name, _) in enumerate(rows) if probe["marker"] in name]
    if len(marks) < n:
        raise SystemExit(f"found {len(marks)} group markers, the probe issues {n}")
    marks = marks[-n:]
    copies = [v for _, v in rows[marks[0] - reps:marks[0]]]
    groups = []
    for g, start in enumerate(marks):
        end = marks[g + 1] if g + 1 < n else len(rows)
        grp = rows[start + 1:end]
        if len(grp) % reps:
            raise SystemExit(f"launch group {g} has {len(grp)} dispatches, not a multiple of {reps}")
        per = len(grp) // reps
        reps_vals = []
        for r in range(reps):
            acc = {}
            for _, vals in grp[r * per:(r + 1) * per]:
                for c, (s, mx) in vals.items():
                    a = acc.get(c, (0.0, 0.0))
                    acc[c] = (a[0] + s, a[1] + mx)
            reps_vals.append(acc)
        groups.append(reps_vals)
    return copies, groups


def _median(reps, counter, which=0):
    import statistics

    return statistics.median(r[counter][which] for r in reps)


def traffic_report(probe_json, fetch_dir, write_dir, prefix=None, groups_prefix=None):
    """Per-launch HBM bytes: each group's median counter value (KiB per launch,
    summed over the kernels a launch issues) scaled by the copy calibration
    (COPY_BYTES / the copy's median). FETCH_SIZE and WRITE_SIZE count L2
    misses to the fabric, so a re-read served by the Infinity Cache counts.
    With `prefix` (e.g. "T2048"), only that block's launches, by launch name;
    with `groups_prefix` (e.g. "c2_"), the groups whose label starts with it."""
    with open(probe_json) as f:
        probe = json.load(f)
    med = {}
    for counter, path in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        copies, groups = _probe_groups(_counter_rows(path), probe)
        med[counter] = [_median(copies, counter)] + [_median(g, counter) for g in groups]
    copy_bytes = probe["copy_bytes"]
    f_scale = copy_bytes / (med["FETCH_SIZE"][0] * 1024)
    w_scale = copy_bytes / (med["WRITE_SIZE"][0] * 1024)
    lines = [f"calibration copy {copy_bytes} B: FETCH_SIZE {med['FETCH_SIZE'][0]:.1f} KiB, "
             f"WRITE_SIZE {med['WRITE_SIZE'][0]:.1f} KiB; scale fetch {f_scale:.4f}, write {w_scale:.4f}"]
    for i, l in enumerate(probe["groups"]):
        if prefix and not l["group"].startswith(prefix + "/"):
            continue
        if groups_prefix and not l["group"].startswith(groups_prefix):
            continue
        fb = med["FETCH_SIZE"][1 + i] * 1024 * f_scale
        wb = med["WRITE_SIZE"][1 + i] * 1024 * w_scale
        label = l["name"] if prefix else l["group"]
        lines.append(f"traffic {label} fetch_bytes={fb:.0f} write_bytes={wb:.0f} hbm_bytes={fb + wb:.0f} "
                     f"algorithmic_bytes={l['bytes']} ratio={(fb + wb) / max(l['bytes'], 1):.3f} "
                     f"summary={l['summary']}")
    print("\n".join(lines))


SIMDS = 1024          # 256 CUs x 4 SIMDs
SHADER_ARRAYS = 32    # 8 XCDs x 4 (rocprofv3 agent info: Array_Count)
ENGINE_GHZ = 2.4


def trace_summary(path, min_calls=20, width=58):
    """Kiln kernels of a rocprofv3 kernel trace (run_kernel_trace.csv) per
    kernel and grid (workgroups x threads): calls, median and minimum
    duration in us. One kernel on one grid can serve two workloads (the same
    tile on two shapes): a group whose sorted durations have a gap larger
    than half its median, with at least min_calls on each side, is printed
    as two rows, split at the largest gap."""
    import csv
    import re
    import statistics

    groups = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if "kh::" not in name:
                continue
            short = re.sub(r"\(kh::.*$", "", re.sub(r"^void kh::\(anonymous namespace\)::", "", name))
            threads = int(r["Workgroup_Size_X"])
            wg = int(r["Grid_Size_X"]) // max(1, threads)
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            groups.setdefault((short, wg, threads), []).append(us)
    print(f"{'kernel':{width}s} {'workgroups x threads':>22s} {'calls':>6s} {'median_us':>10s} {'min_us':>8s}")
    for (k, wg, th), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        if len(v) < min_calls:
            continue
        v = sorted(v)
        gap, i = max(((v[j + 1] - v[j], j) for j in range(len(v) - 1)), default=(0.0, 0))
        split = gap > 0.5 * statistics.median(v) and min(i + 1, len(v) - i - 1) >= min_calls
        for part in ([v[:i + 1], v[i + 1:]] if split else [v]):
            print(f"{k[:width]:{width}s} {f'{wg} x {th}':>22s} {len(part):6d} {statistics.median(part):10.2f} "
                  f"{min(part):8.2f}")


def counter_report(probe_json, dirs):
    """Per-launch SQ counter summary from --pmc passes over --counter-probe
    (each dir one pass). Medians over the repetitions; derived figures:
      mfma_util  = SQ_VALU_MFMA_BUSY_CYCLES / (busy cycles x SIMDs), the busy
                   cycles of the launch being SQ_BUSY_CYCLES / SHADER_ARRAYS
                   (the counter sums the 32 shader arrays; rocprofv3's MfmaUtil
                   divides by GRBM_GUI_ACTIVE instead, which under per-dispatch
                   collection also counts the profiler's own dispatch overhead);
      busy_us    = SQ_BUSY_CYCLES / SHADER_ARRAYS at the 2.4 GHz engine clock;
      mfma_flops = SQ_INSTS_VALU_MFMA_MOPS_{F32,BF16} x 512 (its MfmaFlops*),
                   against the launch's algorithmic flops;
      wait       = SQ_WAIT_ANY / SQ_WAVE_CYCLES (share of wave time waiting
                   on anything: memory counters or a barrier);
      wait_inst  = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (waiting for an
                   instruction's dependencies);
      lds_conf   = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE;
      valu/wave  = SQ_INSTS_VALU / SQ_WAVES, lds/wave = SQ_INSTS_LDS / SQ_WAVES."""
    with open(probe_json) as f:
        probe = json.load(f)
    per_group = [dict() for _ in probe["groups"]]
    for d in dirs:
        _, groups = _probe_groups(_counter_rows(d), probe)
        for i, g in enumerate(groups):
            for c in g[0]:
                if c == "GRBM_GUI_ACTIVE":
                    per_group[i].setdefault(c, _median(g, c, 1))
                else:
                    per_group[i][c] = _median(g, c)

    def ratio(v, a, b):
        return v[a] / v[b] if a in v and b in v and v[b] else None

    def fmt(x, pct=True):
        return "-" if x is None else (f"{100 * x:5.1f}%" if pct else f"{x:7.1f}")

    lines = [f"{'group':34s} {'busy_us':>7s} {'mfma_util':>9s} {'mfma_flops/alg':>14s} {'wait':>7s} {'wait_inst':>9s} "
             f"{'lds_conf':>8s} {'valu/wave':>9s} {'lds/wave':>8s} {'waves':>7s}"]
    for l, v in zip(probe["groups"], per_group):
        busy = v.get("SQ_BUSY_CYCLES", 0.0) / SHADER_ARRAYS
        util = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (busy * SIMDS) if "SQ_VALU_MFMA_BUSY_CYCLES" in v and busy else None
        mops = sum(v.get(c, 0.0) for c in ("SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_MOPS_BF16"))
        fl = mops * 512 / l["flops"] if l["flops"] and mops else None
        lines.append(f"{l['group']:34s} {busy / ENGINE_GHZ / 1e3:7.1f} {fmt(util):>9s} {fmt(fl, False) if fl is None else f'{fl:14.3f}':>14s} "
                     f"{fmt(ratio(v, 'SQ_WAIT_ANY', 'SQ_WAVE_CYCLES')):>7s} "
                     f"{fmt(ratio(v, 'SQ_WAIT_INST_ANY', 'SQ_WAVE_CYCLES')):>9s} "
                     f"{fmt(ratio(v, 'SQ_LDS_BANK_CONFLICT', 'SQ_LDS_IDX_ACTIVE')):>8s} "
                     f"{fmt(ratio(v, 'SQ_INSTS_VALU', 'SQ_WAVES'), False):>9s} "
                     f"{fmt(ratio(v, 'SQ_INSTS_LDS', 'SQ_WAVES'), False):>8s} {v.get('SQ_WAVES', 0):7.0f}")
    lines.append("")
    lines.append("raw medians per launch:")
    for l, v in zip(probe["groups"], per_group):
        lines.append(f"{l['group']}: " + ", ".join(f"{c}={v[c]:.0f}" for c in sorted(v)) + f"  [{l['summary']}]")
    print("\n".join(lines))


def committed_traffic(T, launch):
    """HBM bytes per launch of `launch` from the committed counter summary, if it
    was measured for this very launch (same name and summary), else None."""
    try:
        with open(TRAFFIC_FILE.format(T=T)) as f:
            text = f.read()
    except OSError:
        return None
    for line in text.splitlines():
        if not line.startswith(f"traffic {launch.name} "):
            continue
        fields = dict(kv.split("=", 1) for kv in line.split(" summary=")[0].split()[2:])
        if line.split(" summary=", 1)[1].strip() == launch.summary:
            return int(fields["hbm_bytes"])
    return None


def block_sweep(tokens, autotune, inductor=True):
    """Per T: kiln end to end (copy in, replay, clone out) against eager
    PyTorch-ROCm and torch.compile(mode="reduce-overhead"), and memory per
    call as the reference reports it (benchmarks/bench_gpu.py:163-195): kiln =
    its planned arena + what a call allocates, eager = what a call allocates
    (weights excluded on both sides)."""
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
            # both call paths end to end: copy in + replay + clone out, and the
            # launches straight on the caller's tensors
            ready = c._exe._prepare((x,))
            graph_e2e_ms = ms_per_call(lambda: c._exe._replay(ready))
            direct_ms = ms_per_call(lambda: c._exe._direct(ready))
        kiln_mib = c.report.arena_bytes / 2**20 + peak_mib(c, x)
        eager_mib = peak_mib(model, x)
        ind_ms = inductor_ms(model, x, "reduce-overhead") if inductor else None
        # allow_tf32 (three-pass bf16 GEMMs): reported beside, never the headline
        ct = kiln.compile(model, (x,), device="cuda", autotune=autotune, allow_tf32=True)
        with torch.no_grad():
            ref64 = model.double()(x.double())
            model.float()
            tf_err = ((ct(x).double() - ref64).abs().max() / ref64.abs().max()).item()
            assert tf_err <= 5e-5, f"block T={T} allow_tf32: error {tf_err:.2e} of the output scale"
            tf_ms = ms_per_call(lambda: ct(x))
        # the bf16-input / fp32-accumulate variant (matmul_precision="bf16"):
        # reported beside, with its error against float64
        cb = kiln.compile(model, (x,), device="cuda", autotune=autotune, matmul_precision="bf16")
        with torch.no_grad():
            bf_err = ((cb(x).double() - ref64).abs().max() / ref64.abs().max()).item()
            assert bf_err <= 2e-2, f"block T={T} bf16: error {bf_err:.2e} of the output scale"
            bf_ms = ms_per_call(lambda: cb(x))
        out[str(T)] = {"kiln_ms": round(k_ms, 4), "eager_ms": round(e_ms, 4), "replay_ms": round(replay_ms, 4),
                       "call_mode": c._exe.mode, "graph_e2e_ms": round(graph_e2e_ms, 4),
                       "direct_ms": round(direct_ms, 4), "launches": c.report.lowering["launches"],
                       "inductor_ms": round(ind_ms, 4) if ind_ms else None,
                       "speedup": round(e_ms / k_ms, 3), "tflops": round(block_flops(T) / k_ms / 1e9, 2),
                       "arena_mib": round(c.report.arena_bytes / 2**20, 2),
                       "kiln_mib": round(kiln_mib, 2), "eager_mib": round(eager_mib, 2),
                       "allow_tf32_ms": round(tf_ms, 4), "allow_tf32_error_of_scale": float(f"{tf_err:.2e}"),
                       "bf16_ms": round(bf_ms, 4), "bf16_error_of_scale": float(f"{bf_err:.2e}"),
                       "bf16_launches": cb.report.lowering["launches"]}
        log(f"block T={T}: kiln {k_ms:.4f} ms ({c._exe.mode}; graph path {graph_e2e_ms:.4f}, direct {direct_ms:.4f}, "
            f"replay alone {replay_ms:.4f}), eager {e_ms:.4f} ms, "
            f"inductor {ind_ms if ind_ms else float('nan'):.4f} ms, allow_tf32 {tf_ms:.4f} ms, bf16 {bf_ms:.4f} ms, "
            f"MiB kiln {kiln_mib:.1f} / eager {eager_mib:.1f}")
    return out


GEMM_SHAPES = [(2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768), (128, 768, 3072),
               (1, 3072, 768)]


def gemm_sweep(autotune):
    """The benchmark's nn.Linear sweep (bias epilogue), fp32 and, reported
    separately, the bf16-input / fp32-accumulate variant. TFLOP/s from GPU time
    of a 20-call graph replay; eager torch beside each (bf16 with inputs
    already cast, its best case). bf16 also reports the fraction of the
    attainable bound min(bf16 peak, AI x 8 TB/s), AI from the algorithmic
    bytes (fp32 X, bf16 W, fp32 bias and output)."""
    import torch
    import torch.nn.functional as F

    import kiln
    from models.transformer import gpt2_init_

    out = {"fp32": {}, "bf16": {}, "bf16x3": {}}
    for m, n, k in GEMM_SHAPES:
        torch.manual_seed(0)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=1).eval().cuda()
        x = torch.randn(m, k, device="cuda")
        flops = 2 * m * n * k
        c = kiln.compile(lin, (x,), device="cuda", autotune=autotune, cuda_graphs=False)
        with torch.no_grad():
            torch.testing.assert_close(c(x), lin(x), rtol=1e-4, atol=1e-5)
            outs = [torch.empty(m, n, device="cuda")]
            kms = graph_ms(lambda: c._exe.run_into([x], outs))
            ems = graph_ms(lambda: lin(x))
        out["fp32"][f"{m}x{n}x{k}"] = {"kiln_tflops": round(flops / kms / 1e9, 2),
                                       "torch_tflops": round(flops / ems / 1e9, 2), "kiln_us": round(kms * 1e3, 2),
                                       "frac_of_fp32_peak": round(flops / kms / 1e9 / FP32_PEAK_TFLOPS, 3)}
        log(f"gemm fp32 {m}x{n}x{k}: kiln {flops / kms / 1e9:.1f} TFLOP/s, torch {flops / ems / 1e9:.1f}")
        cb = kiln.compile(lin, (x,), device="cuda", autotune=autotune, cuda_graphs=False, matmul_precision="bf16")
        xb, wb, bb = x.bfloat16(), lin.weight.detach().bfloat16().contiguous(), lin.bias.detach().bfloat16()
        with torch.no_grad():
            ref = lin(x)
            got = cb(x)
            err = ((got - ref).abs().max() / ref.abs().max()).item()
            assert err <= 2e-2, f"bf16 GEMM {m}x{n}x{k}: error {err:.2e} of the output scale"
            bms = graph_ms(lambda: cb._exe.run_into([x], outs))
            tms = graph_ms(lambda: F.linear(xb, wb, bb))
        nbytes = 4 * m * k + 2 * k * n + 4 * n + 4 * m * n
        attainable = min(BF16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)
        tf = flops / bms / 1e9
        out["bf16"][f"{m}x{n}x{k}"] = {"kiln_tflops": round(tf, 2), "torch_tflops": round(flops / tms / 1e9, 2),
                                       "kiln_us": round(bms * 1e3, 2), "error_of_scale": float(f"{err:.2e}"),
                                       "attainable_tflops": round(attainable, 1),
                                       "frac_of_attainable": round(tf / attainable, 3)}
        log(f"gemm bf16 {m}x{n}x{k}: kiln {tf:.1f} TFLOP/s ({tf / attainable:.1%} of attainable "
            f"{attainable:.0f}), torch-bf16 {flops / tms / 1e9:.1f}")
        # allow_tf32: the three-pass bf16 GEMM (fp32-class error, see
        # tests/test_gpu_bf16x3.py); error against float64 of the fp32 inputs
        cx = kiln.compile(lin, (x,), device="cuda", autotune=autotune, cuda_graphs=False, allow_tf32=True)
        with torch.no_grad():
            ref64 = x.double() @ lin.weight.double().t() + lin.bias.double()
            err = ((cx(x).double() - ref64).abs().max() / ref64.abs().max()).item()
            assert err <= 5e-5, f"bf16x3 GEMM {m}x{n}x{k}: error {err:.2e} of the output scale"
            xms = graph_ms(lambda: cx._exe.run_into([x], outs))
        out["bf16x3"][f"{m}x{n}x{k}"] = {"kiln_tflops": round(flops / xms / 1e9, 2), "kiln_us": round(xms * 1e3, 2),
                                         "error_of_scale": float(f"{err:.2e}"),
                                         "vs_fp32": round(kms / xms, 3)}
        log(f"gemm bf16x3 {m}x{n}x{k}: kiln {flops / xms / 1e9:.1f} TFLOP/s ({kms / xms:.2f}x the fp32 path), "
            f"error {err:.1e} of the output scale")
    return out


def linear_gelu(autotune):
    """The benchmark's C1: nn.Linear(768, 3072) + bias + GELU at [128, 768], with
    nn.GELU's default (erf) form and the tanh form the Block uses; GPU time of
    a 20-call graph replay, eager torch beside each."""
    import torch

    import kiln
    from models.transformer import gpt2_init_

    m, k, n = 128, 768, 3072
    flops = 2 * m * n * k
    out = {}
    for approx in ("none", "tanh"):
        torch.manual_seed(0)
        model = torch.nn.Sequential(gpt2_init_(torch.nn.Linear(k, n), seed=1),
                                    torch.nn.GELU(approximate=approx)).eval().cuda()
        x = torch.randn(m, k, device="cuda")
        c = kiln.compile(model, (x,), device="cuda", autotune=autotune, cuda_graphs=False)
        with torch.no_grad():
            torch.testing.assert_close(c(x), model(x), rtol=1e-4, atol=1e-5)
            outs = [torch.empty(m, n, device="cuda")]
            kms = graph_ms(lambda: c._exe.run_into([x], outs))
            ems = graph_ms(lambda: model(x))
        name = f"linear_gelu_{'erf' if approx == 'none' else 'tanh'}_{m}x{k}x{n}"
        out[name] = {"kiln_us": round(kms * 1e3, 2), "eager_us": round(ems * 1e3, 2),
                     "kiln_tflops": round(flops / kms / 1e9, 2), "launches": c.report.lowering["launches"]}
        log(f"{name}: kiln {kms * 1e3:.2f} us ({flops / kms / 1e9:.1f} TFLOP/s, "
            f"{c.report.lowering['launches']} launch), eager {ems * 1e3:.2f} us")
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
        # a device copy of the same shape (the same bytes read and written,
        # one launch), hot and cold the same way: what any single launch of
        # this size can reach on this box
        copy_hot = graph_ms(lambda: y.copy_(x))

        def copy_step():
            i = state["i"] % n
            state["i"] += 1
            ys[i].copy_(xs[i])

        copy_cold = graph_ms(copy_step, repeats=n, rounds=3)
        with torch.no_grad():
            eager = graph_ms(lambda: fn(x))
        out[name] = {"kiln_hot_us": round(hot * 1e3, 2), "kiln_cold_us": round(cold * 1e3, 2),
                     "eager_hot_us": round(eager * 1e3, 2),
                     "copy_hot_us": round(copy_hot * 1e3, 2), "copy_cold_us": round(copy_cold * 1e3, 2),
                     "hot_gbs": round(nbytes / hot / 1e6, 1), "cold_gbs": round(nbytes / cold / 1e6, 1),
                     "cold_hbm_frac": round(nbytes / cold / 1e6 / HBM_PEAK_GBS, 3),
                     "cold_of_copy": round(copy_cold / cold, 3), "hot_of_copy": round(copy_hot / hot, 3),
                     "bytes": nbytes}
        log(f"{name}: hot {hot * 1e3:.2f} us ({nbytes / hot / 1e6:.0f} GB/s), cold {cold * 1e3:.2f} us "
            f"({nbytes / cold / 1e6:.0f} GB/s, {copy_cold / cold:.2f} of a copy's {copy_cold * 1e3:.2f} us), "
            f"eager {eager * 1e3:.2f} us")
        del xs, ys
        torch.cuda.empty_cache()
    # the same kernels at 1.5 GiB of traffic per call (six times the Infinity
    # Cache): HBM bandwidth against the 8 TB/s peak and against a plain
    # device copy of the same bytes
    scale = [
        ("bias_gelu_65536x3072", work[0][1], (65536, 3072)),
        ("layernorm_262144x768", ln, (262144, 768)),
        ("softmax_48x2048x2048", work[2][1], (48, 2048, 2048)),
    ]
    for name, fn, shape in scale:
        x = torch.randn(*shape, device="cuda")
        nbytes = 2 * x.numel() * 4
        c = kiln.compile(fn, (x,), device="cuda", cuda_graphs=False)
        y = torch.empty_like(x)
        c._exe.run_into([x], [y])
        with torch.no_grad():
            torch.testing.assert_close(y, fn(x), rtol=1e-4, atol=1e-5)
            y.copy_(x)  # warm the copy path too
            ms = events_ms(lambda: c._exe.run_into([x], [y]), 10)
            copy = events_ms(lambda: y.copy_(x), 10)
            eager = events_ms(lambda: fn(x), 10)
        out[name] = {"kiln_us": round(ms * 1e3, 1), "copy_us": round(copy * 1e3, 1), "eager_us": round(eager * 1e3, 1),
                     "gbs": round(nbytes / ms / 1e6, 1), "hbm_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 3),
                     "of_copy": round(copy / ms, 3), "bytes": nbytes}
        log(f"{name}: {ms * 1e3:.1f} us ({nbytes / ms / 1e6:.0f} GB/s, {nbytes / ms / 1e6 / HBM_PEAK_GBS:.2f} of peak, "
            f"{copy / ms:.2f} of a copy), eager {eager * 1e3:.1f} us")
        del x, y, c
        torch.cuda.empty_cache()
    return out


def stack_bench(autotune):
    import torch

    import kiln
    from models.transformer import Stack, gpt2_init_

    out = {}
    # decode_1_chain: the same decode with its 48 GEMVs as one persistent
    # launch (gemv_chains, opt-in), measured beside the default;
    # decode_1_bf16: the decode on the bf16 weight copies (162.5 MiB instead
    # of 324.5), checked against eager at the bf16 tolerance
    for name, T, chains, prec in (("prefill_1024", 1024, False, "fp32"), ("decode_1", 1, False, "fp32"),
                                  ("decode_1_chain", 1, True, "fp32"), ("decode_1_bf16", 1, False, "bf16")):
        torch.manual_seed(0)
        model = gpt2_init_(Stack(12, 768, 12, T), seed=0).eval().cuda()
        x = torch.randn(T, 768, device="cuda")
        c = kiln.compile(model, (x,), device="cuda", autotune=autotune, gemv_chains=chains, matmul_precision=prec)
        with torch.no_grad():
            ref = model(x)
            if prec == "fp32":
                torch.testing.assert_close(c(x), ref, rtol=1e-4, atol=1e-5)
            else:
                assert float((c(x) - ref).abs().max()) <= 2e-2 * float(ref.abs().max())
            k_ms = ms_per_call(lambda: c(x))
            e_ms = ms_per_call(lambda: model(x))
        flops = 12 * block_flops(T)
        out[name] = {"kiln_ms": round(k_ms, 4), "eager_ms": round(e_ms, 4), "tflops": round(flops / k_ms / 1e9, 2),
                     "launches": c.report.lowering["launches"],
                     "kernel_launches": c.report.lowering["kernel_launches"]}
        if T == 1:   # the algorithmic bytes of every launch (weights once each), per call
            nbytes = sum(launch.bytes for launch in c._exe.program.launches)
            out[name]["bytes"] = nbytes
            out[name]["gbs"] = round(nbytes / k_ms / 1e6, 1)
        log(f"stack {name}: kiln {k_ms:.4f} ms ({c.report.lowering['kernel_launches']} kernel launches), "
            f"eager {e_ms:.4f} ms" + (f", {out[name]['gbs']} GB/s of {out[name]['bytes'] / 1e6:.1f} MB" if T == 1 else ""))
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_ms_per_call(fn, x, min_time=1.0):
    """The reference's CPU timing (benchmarks/bench_block.py:41-54): one
    warm-up call, as many calls as fit in min_time / 3, then the best of 3
    rounds of that many calls."""
    import torch

    with torch.no_grad():
        fn(x)
        start, calls = time.perf_counter(), 0
        while time.perf_counter() - start < min_time / 3:
            fn(x)
            calls += 1
        calls = max(calls, 1)
        best = float("inf")
        for _ in range(3):
            start = time.perf_counter()
            for _ in range(calls):
                fn(x)
            best = min(best, (time.perf_counter() - start) / calls)
    return best * 1e3


def cpu_baseline(T, oracle_line=True):
    """The C oracle (oracle/kiln_oracle.c: the CPU port of the reference's
    algorithm for the block, float64 naive loops, one thread) on the headline
    block with the GPU run's weights and input, twice (~12 s): the `port`
    baseline. Beside it, eager PyTorch CPU fp32 on the same block at 1 thread
    (the reference's convention, benchmarks/bench_block.py:61) and at every
    core this process may use (capped by OMP_NUM_THREADS, the box's CPU
    share). The reference's own CPU path (MLIR -> LLVM JIT) cannot be built
    here: no MLIR bindings, an empty LLVM pin, a network-only build script."""
    import torch

    from models.transformer import Block, gpt2_init_

    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768, generator=torch.Generator().manual_seed(1))
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    before = torch.get_num_threads()
    try:
        torch.set_num_threads(1)
        one = cpu_ms_per_call(model, x)
        torch.set_num_threads(cores)
        many = cpu_ms_per_call(model, x)
    finally:
        torch.set_num_threads(before)
    log(f"cpu baseline: eager PyTorch CPU fp32 block T={T}: {one:.1f} ms at 1 thread, {many:.1f} ms at {cores}")
    eager = {"value": round(many, 2), "unit": "ms", "cores": cores,
             "impl": "eager PyTorch CPU fp32 (torch " + torch.__version__ + ")",
             "sample": f"one full GPT-2-small block forward at T={T}, best of 3 rounds after calibration "
                       f"(reference benchmarks/bench_block.py:41-54)",
             "single_thread": {"value": round(one, 2), "unit": "ms", "cores": 1}}
    out = {"value": None, "unit": "ms", "cores": 1, "kind": "port",
           "impl": "oracle/kiln_oracle.c: the C port of the reference's block algorithm, float64 naive loops",
           "cpu_model": cpu_model(), "eager_pytorch_cpu": eager,
           "reference_cpu_path": "unavailable: MLIR Python bindings absent, LLVM pin empty, network-only build"}
    if oracle_line:
        import oracle

        params = {k: v.numpy() for k, v in model.state_dict().items()}
        oracle.lib()
        runs = []
        for _ in range(2):
            t0 = time.perf_counter()
            oracle.block(x.numpy(), params, 12)
            runs.append((time.perf_counter() - t0) * 1e3)
        out["value"] = round(min(runs), 1)
        out["sample"] = (f"one full GPT-2-small block forward at T={T} (the headline workload, same seeded weights and "
                         f"input), best of {len(runs)} runs ({sum(runs) / 1e3:.1f} s of CPU work)")
        log(f"cpu baseline: C oracle (float64, 1 thread) block T={T}: {out['value']:.1f} ms")
    return out


def mfma_probe():
    """Shader cycles per 32x32x2 fp32 MFMA per SIMD under the library's
    kh_probe_mfma_valu: MFMA-only streams, then MFMAs with VALU work in the
    same wave (one and two waves per SIMD)."""
    import ctypes
    from kiln.hip import lib as kl

    lib = kl.load()
    out = (ctypes.c_double * 2)()
    log("MFMA / VALU issue probe (32x32x2 fp32 MFMA = 64 matrix-core cycles at full rate):")
    log("  waves/SIMD chains group valu   cycles/MFMA   clock GHz")
    for wps in (1, 2):
        for c, g, v in ((1, 1, 0), (2, 1, 0), (1, 1, 1), (1, 1, 2), (1, 1, 4), (2, 1, 2), (4, 1, 2), (8, 1, 2),
                        (1, 4, 8), (1, 8, 16), (2, 8, 16), (1, 32, 64)):
            kl.check(lib.kh_probe_mfma_valu(c, g, v, wps, out), "kh_probe_mfma_valu")
            log(f"  {wps:10d} {c:6d} {g:5d} {v:4d} {out[0]:13.1f} {out[1]:11.3f}")


def attention_timeline():
    """Per-workgroup timeline of the 32-query attention kernel on the GPT-2
    block's T = 2048 operands (the QKV product's [T, 2304] output read as
    q, k, v), from kh_probe_attn_timeline: makespan, per-block cycles of the
    longest workgroups, the shader clock, how many workgroups ran per CU and
    when the CUs went idle."""
    import ctypes
    import numpy as np
    import torch
    from kiln.hip import lib as kl

    lib = kl.load()
    T, DH = 2048, 64
    torch.manual_seed(0)
    qkv = torch.randn(T, 3 * 768, device="cuda")
    out = torch.empty(T, 768, device="cuda")
    st = (ctypes.c_int64 * 8)(DH, 2304, DH, 2304, DH, 2304, DH, 768)
    stream = torch.cuda.current_stream().cuda_stream
    log("attention timeline (kh_probe_attn_timeline, causal, head dim 64, GPT-2 QKV layout):")
    for heads, nw in ((12, 4), (12, 8), (4, 4), (4, 8)):
        nq = (T + 31) // 32
        rec = torch.zeros(heads * nq * nw * 8, dtype=torch.int64, device="cuda")
        q, k, v = qkv[:, :768], qkv[:, 768:1536], qkv[:, 1536:]
        for _ in range(20):  # the last run's records are kept
            kl.check(lib.kh_probe_attn_timeline(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), heads, T,
                                                T, st, nw, 0.125, rec.data_ptr(), stream), "kh_probe_attn_timeline")
        torch.cuda.synchronize()
        r = rec.cpu().numpy().reshape(heads * nq, nw, 8).view(np.uint64).astype(np.float64)
        t0, t1, t2 = r[:, :, 0].min(1), r[:, :, 1], r[:, :, 2].max(1)
        base = t0.min()
        span = (t2.max() - base) * 0.01
        blocks = r[:, :, 7].max(1)
        ghz = (r[:, :, 4] - r[:, :, 3]) / ((r[:, :, 2] - r[:, :, 0]) * 10.0)
        hw = r[:, 0, 5].astype(np.int64)
        cu_id = (r[:, 0, 6].astype(np.int64) & 15) * 4096 + ((hw >> 13) & 7) * 512 + ((hw >> 12) & 1) * 256 + ((hw >> 8) & 15)
        longest = blocks >= blocks.max() - 1
        dur = (t2 - t0) * 0.01
        cyc = ((r[:, :, 4] - r[:, :, 3]).max(1))[longest] / blocks[longest]
        per_cu = {}
        idle = {}
        for g in range(len(t0)):
            per_cu[cu_id[g]] = per_cu.get(cu_id[g], 0) + 1
            idle[cu_id[g]] = max(idle.get(cu_id[g], 0.0), (t2[g] - base) * 0.01)
        counts = {}
        for n in per_cu.values():
            counts[n] = counts.get(n, 0) + 1
        iv = np.array(sorted(idle.values()))
        grid = np.linspace(0, span, 9)
        active = [int(((t0 - base) * 0.01 <= t).sum() - ((t2 - base) * 0.01 <= t).sum()) for t in grid]
        log(f"  {heads} heads, {nw} waves per workgroup: {len(t0)} workgroups on {len(per_cu)} CUs, makespan "
            f"{span:.1f} us, shader clock median {np.median(ghz):.2f} GHz")
        log(f"    longest workgroups ({int(blocks.max())} key blocks per wave): {np.median(dur[longest]):.1f} us, "
            f"{np.median(cyc):.0f} shader cycles per key block per wave (64 MFMAs = 4096 matrix-core cycles)")
        log(f"    workgroups per CU: {dict(sorted(counts.items()))}; CUs idle from {iv.min():.1f} us (first), "
            f"{np.median(iv):.1f} (median), {iv.max():.1f} (last)")
        log("    workgroups running: " + "  ".join(f"{t:.0f}us:{n}" for t, n in zip(grid, active)))


def main():
    args = parse()
    if args.traffic_report:
        if args.traffic_groups:
            traffic_report(*args.traffic_report, groups_prefix=args.traffic_groups)
        else:
            traffic_report(*args.traffic_report, prefix=f"T{args.tokens}")
        return
    if args.counter_report:
        counter_report(args.counter_report[0], args.counter_report[1:])
        return
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        sys.exit("bench.py needs an MI355X (no ROCm GPU visible)")
    from kiln.hip import lib as kl
    from kiln.hip.interpret import refuse

    refuse("bench.py")

    if args.counter_probe:
        counter_probe(args)
        return
    if args.probes:
        mfma_probe()
        attention_timeline()
        return
    torch.manual_seed(0)
    info = kl.device_info() if kl.load() else {}
    extra = {}
    compiled, model, x, err = prepare_headline(args)
    if not args.quick:
        # untimed sections first: the headline's timed steps then follow GPU
        # work directly and run at the clocks it brought up (the block sweep,
        # ending on the T = 2048 block, goes last)
        extra["gemm"] = gemm_sweep(not args.no_autotune)
        extra["linear_gelu"] = linear_gelu(not args.no_autotune)
        extra["fused_ops"] = fused_ops()
        extra["stack"] = stack_bench(not args.no_autotune)
        extra["block"] = block_sweep([128, 512, 1024, 2048], not args.no_autotune, not args.no_inductor)
    ms = time_headline(args, compiled, x)
    log(f"headline: block T={args.tokens}: {ms:.4f} ms/step over {args.steps} steps (max err {err:.2e})")
    roofline, prof = dominant_kernel_roofline(compiled, x, args.tokens)
    log("per-launch ms: " + ", ".join(f"{n}={t:.4f}" for n, t in prof))
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.tokens)
    line = {
        "metric": "GPT-2 block latency ms @128-2048 tok; GEMM TFLOP/s; fused-op GB/s (1 GPU)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (seeded N(0,1) input, random-init N(0,0.02) weights)",
        "config": {"workload": f"gpt2_small_block_T{args.tokens}", "tokens": args.tokens, "d_model": 768,
                   "heads": 12, "parallelism": "none (1 GPU)", "call_mode": compiled._exe.mode,
                   "launches": compiled.report.lowering["launches"]},
        "roofline": roofline, "cpu_baseline": cpu,
        "device": info, "per_launch_ms": {n: round(t, 5) for n, t in prof}, **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
