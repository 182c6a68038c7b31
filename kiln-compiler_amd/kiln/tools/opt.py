"""kiln-opt: apply passes to textual IR, like mlir-opt.

    python -m kiln.tools.opt input.kir --passes=freeze,const-fold,canonicalize
    python -m kiln.tools.opt input.kir --passes=fusion,buffer-assign,memory-plan
    python -m kiln.tools.opt input.kir --pipeline=default --emit=plan

Reads a file (or stdin for "-") and prints the resulting IR, or with
``--emit=plan`` the lowered HIP launch plan listing. Pass names are Kiln's
(the reference's kiln/tools/opt.py:27-51) without the CPU-only ``schedule``;
the FileCheck fixtures in tests/lit run through this tool.
"""

from __future__ import annotations

import argparse
import sys


def pass_registry() -> dict:
    """{pass name: factory}."""
    from kiln.passes.buffers import BufferAssignment
    from kiln.passes.freeze import ConstantFold, FreezeParameters
    from kiln.passes.fusion import Fusion
    from kiln.passes.memory_plan import MemoryPlan
    from kiln.passes.partition import OneOpPerKernel
    from kiln.passes.simplify import CSE, DCE, Canonicalize

    factories = [Canonicalize, CSE, DCE, FreezeParameters, ConstantFold, OneOpPerKernel, Fusion,
                 BufferAssignment, MemoryPlan]
    registry = {f.name: f for f in factories}
    registry["buffer-assign"] = BufferAssignment
    registry["memory-plan-naive"] = lambda: MemoryPlan(reuse=False)
    return registry


def make_pass(name: str):
    registry = pass_registry()
    if name not in registry:
        raise SystemExit(f"kiln-opt: unknown pass '{name}' (known: {', '.join(sorted(registry))})")
    return registry[name]()


def pipeline(args) -> list:
    from kiln.api import Options, build_passes

    if args.pipeline:
        return build_passes(Options() if args.pipeline == "default" else Options.none())
    return [make_pass(name.strip()) for name in args.passes.split(",") if name.strip()]


def main(argv=None) -> int:
    from kiln.ir.parser import ParseError, parse
    from kiln.passes.manager import PassManager

    cli = argparse.ArgumentParser(prog="kiln-opt", description=__doc__.splitlines()[0])
    cli.add_argument("input", nargs="?", default="-")
    cli.add_argument("--passes", default="", help="comma-separated pass names, run in order")
    cli.add_argument("--pipeline", choices=["default", "none"], default=None,
                     help="kiln.compile's pipeline with every optimisation on (default) or off (none)")
    cli.add_argument("--emit", choices=["ir", "plan"], default="ir")
    cli.add_argument("--print-ir-after-all", action="store_true")
    args = cli.parse_args(argv)

    source = sys.stdin if args.input == "-" else open(args.input)
    with source:
        text = source.read()
    try:
        graph = parse(text)
    except ParseError as err:
        print(f"kiln-opt: {err}", file=sys.stderr)
        return 1
    PassManager(pipeline(args), print_after_all=args.print_ir_after_all).run(graph)
    if args.emit == "plan":
        from kiln.hip.lowering import lower_graph

        sys.stdout.write(lower_graph(graph).source)
    else:
        print(graph)
    return 0


if __name__ == "__main__":
    sys.exit(main())
