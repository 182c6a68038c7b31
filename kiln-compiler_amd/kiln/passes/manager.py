"""Pass driver.

A pass is an object with a ``name`` and ``run(graph)`` that rewrites the graph
in place and may return a dict of statistics (Kiln's pass interface, the
reference's kiln/passes/manager.py:11-41). ``PassManager`` runs a list of
them, keeping one ``PassRecord`` per execution; ``timings`` (seconds summed
per pass name) and ``stats`` (the latest non-empty statistics per name) are
views of that history, which is what ``Report`` shows.
"""

from __future__ import annotations

import sys
import time
from dataclasses import dataclass

from kiln.ir.core import Graph, verify


class Pass:
    name = "pass"

    def run(self, graph: Graph):
        """Rewrite ``graph`` in place; return a dict of statistics or None."""
        raise NotImplementedError(f"{type(self).__name__}.run")


@dataclass
class PassRecord:
    name: str
    seconds: float
    stats: dict | None


class PassManager:
    def __init__(self, passes, print_after_all=False, verify_each=True, stream=None):
        self.passes = list(passes)
        self.print_after_all = print_after_all
        self.verify_each = verify_each
        self.stream = stream
        self.history: list = []

    def run(self, graph: Graph) -> Graph:
        for p in self.passes:
            started = time.perf_counter()
            result = p.run(graph)
            self.history.append(PassRecord(p.name, time.perf_counter() - started, result or None))
            if self.verify_each:
                verify(graph)
            if self.print_after_all:
                print(f"// ----- IR after {p.name} -----", graph, sep="\n", file=self.stream or sys.stdout)
        return graph

    @property
    def timings(self) -> dict:
        total = {}
        for rec in self.history:
            total[rec.name] = total.get(rec.name, 0.0) + rec.seconds
        return total

    @property
    def stats(self) -> dict:
        return {rec.name: rec.stats for rec in self.history if rec.stats}
