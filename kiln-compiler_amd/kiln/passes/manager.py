"""Pass infrastructure (contract of the reference's kiln/passes/manager.py:11-41):
``Pass.run(graph) -> stats | None`` and a ``PassManager`` that times each pass,
records its statistics, verifies the IR after it and can dump the IR."""

from __future__ import annotations

import time

from kiln.ir.core import Graph, verify


class Pass:
    name = "pass"

    def run(self, graph: Graph):
        """Transform ``graph`` in place; may return a dict of statistics."""
        raise NotImplementedError


class PassManager:
    def __init__(self, passes, print_after_all=False, verify_each=True):
        self.passes = list(passes)
        self.print_after_all = print_after_all
        self.verify_each = verify_each
        self.timings: dict = {}
        self.stats: dict = {}

    def run(self, graph: Graph) -> Graph:
        for p in self.passes:
            t0 = time.perf_counter()
            stats = p.run(graph)
            self.timings[p.name] = self.timings.get(p.name, 0.0) + (time.perf_counter() - t0)
            if stats:
                self.stats[p.name] = stats
            if self.verify_each:
                verify(graph)
            if self.print_after_all:
                print(f"// ----- IR after {p.name} -----\n{graph}")
        return graph
