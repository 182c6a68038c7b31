"""kiln-opt: run Kiln passes on textual IR (the analogue of mlir-opt).

    python -m kiln.tools.opt input.kir --passes=freeze,const-fold,canonicalize
    python -m kiln.tools.opt input.kir --passes=fusion,buffer-assign,memory-plan
    python -m kiln.tools.opt input.kir --pipeline=default --emit=plan

Reads a file or stdin ("-"), writes the resulting IR (or, with --emit=plan,
the lowered HIP launch plan) to stdout. Same pass names as the reference tool
(kiln/tools/opt.py:27-51) minus the CPU-only ``schedule``; the FileCheck tests
in tests/lit run through it.
"""

from __future__ import annotations

import argparse
import sys


def make_pass(name):
    from kiln.passes.buffers import BufferAssignment
    from kiln.passes.freeze import ConstantFold, FreezeParameters
    from kiln.passes.fusion import Fusion
    from kiln.passes.memory_plan import MemoryPlan
    from kiln.passes.partition import OneOpPerKernel
    from kiln.passes.simplify import CSE, DCE, Canonicalize

    table = {
        "canonicalize": Canonicalize, "cse": CSE, "dce": DCE, "freeze": FreezeParameters,
        "const-fold": ConstantFold, "partition": OneOpPerKernel, "fusion": Fusion,
        "buffer-assign": BufferAssignment, "memory-plan": MemoryPlan,
        "memory-plan-naive": lambda: MemoryPlan(reuse=False),
    }
    if name not in table:
        raise SystemExit(f"kiln-opt: unknown pass '{name}' (known: {', '.join(table)})")
    return table[name]()


def main(argv=None):
    from kiln.api import Options, build_passes
    from kiln.ir.parser import ParseError, parse
    from kiln.passes.manager import PassManager

    p = argparse.ArgumentParser(prog="kiln-opt", description=__doc__.splitlines()[0])
    p.add_argument("input", nargs="?", default="-")
    p.add_argument("--passes", default="", help="comma-separated pass names")
    p.add_argument("--pipeline", choices=["default", "none"], default=None)
    p.add_argument("--emit", choices=["ir", "plan"], default="ir")
    p.add_argument("--print-ir-after-all", action="store_true")
    args = p.parse_args(argv)

    text = sys.stdin.read() if args.input == "-" else open(args.input).read()
    try:
        graph = parse(text)
    except ParseError as e:
        print(f"kiln-opt: {e}", file=sys.stderr)
        return 1
    if args.pipeline == "default":
        passes = build_passes(Options())
    elif args.pipeline == "none":
        passes = build_passes(Options.none())
    else:
        passes = [make_pass(n) for n in args.passes.split(",") if n]
    PassManager(passes, print_after_all=args.print_ir_after_all).run(graph)
    if args.emit == "plan":
        from kiln.hip.lowering import lower_graph

        print(lower_graph(graph).source, end="")
    else:
        print(graph)
    return 0


if __name__ == "__main__":
    sys.exit(main())
