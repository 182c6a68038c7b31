"""Regenerate the shipped tuning table (kiln/hip/tuned_configs.json).

    python -m kiln.hip.tune_shipped [--out PATH]

Runs the measured autotuner (kiln.hip.autotune.GPUAutotuner, no cache, no
shipped table) on one MI355X for every GEMM shape of the GPT-2-small block at
T = 128, 512, 1024 and 2048 tokens, the 12-layer stack and the benchmark GEMM
sweep, in fp32 and bf16 (the block products also as "bf16+a16": timed reading a
bf16 A operand, as a bf16 plan stores it), and writes the winners keyed like
the on-disk cache (device|CUs|precision|BxMxNxK). The table is what makes a plan the same on
every MI355X: compiled models look their shapes up there before measuring.
"""

from __future__ import annotations

import argparse
import json
import sys

from kiln.hip import autotune

# block products (qkv, attention projection, MLP up, MLP down) at each token
# count: in a bf16 plan their A operands come from a LayerNorm, the attention
# or the MLP-up product, which store them as bf16 for the configurations that
# read A that way ("bf16+a16" entries); in a three-pass plan, as pair words
# ("bf16x3+a16")
BLOCK = sorted((t, n, k) for t in (128, 512, 1024, 2048) for n, k in ((2304, 768), (768, 768), (3072, 768), (768, 3072)))

SHAPES = sorted({
    # GPT-2 block: qkv, attention projection, MLP up, MLP down, at each token count
    *((t, n, k) for t in (128, 512, 1024, 2048) for n, k in ((2304, 768), (768, 768), (3072, 768), (768, 3072))),
    # the benchmark GEMM sweep (the M = 1 decode shape is a GEMV in fp32)
    (2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768), (128, 768, 3072), (1, 3072, 768),
    (1, 2304, 768), (1, 768, 768), (1, 768, 3072),
})


def warm_up(seconds=1.0):
    """Run large products until the GPU's clocks are up, so the first shape
    is not timed on a cold GPU."""
    import time

    import torch

    from kiln.hip.runtime import device

    x = torch.randn(8192, 8192, device=device())
    end = time.perf_counter() + seconds
    while time.perf_counter() < end:
        for _ in range(10):
            x @ x
        torch.cuda.synchronize()


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--out", default=str(autotune.SHIPPED_PATH))
    p.add_argument("--precision", nargs="+", choices=("fp32", "bf16", "bf16+a16", "bf16x3", "bf16x3+a16"), default=None,
                   help="re-tune only these precisions and keep the table's other entries")
    p.add_argument("--max-m", type=int, default=None,
                   help="re-tune only shapes with at most this many rows and keep the table's other entries")
    args = p.parse_args(argv)
    warm_up()
    shapes = [s for s in SHAPES if args.max_m is None or s[0] <= args.max_m]
    precisions = args.precision or ("fp32", "bf16", "bf16+a16", "bf16x3", "bf16x3+a16")
    table = {}
    if args.precision or args.max_m is not None:
        retuned = {(p_, f"1x{m}x{n}x{k}") for p_ in precisions for m, n, k in shapes}
        table = {key: v for key, v in autotune.shipped_configs().items()
                 if (key.split("|")[-2], key.split("|")[-1]) not in retuned}
    for precision in precisions:
        a16 = precision.endswith("+a16")
        base = precision.split("+")[0]
        tuner = autotune.GPUAutotuner(precision=base, use_cache=False, use_shipped=False)
        device = tuner.device_key()
        for m, n, k in shapes:
            if a16 and (m, n, k) not in BLOCK:
                continue
            entry = tuner.tune(1, m, n, k, autotune.default_config_for(1, m, n, k, precision=base), a16=a16)
            if entry["candidates"]:
                table[f"{device}|{precision}|1x{m}x{n}x{k}"] = entry
            print(f"{precision} {m}x{n}x{k}: {entry['config']} {entry['tflops']} TFLOP/s", flush=True)
    with open(args.out, "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {len(table)} entries to {args.out}")


if __name__ == "__main__":
    sys.exit(main())
