"""One op per kernel: the ``fusion=False`` ablation baseline
(reference: kiln/passes/partition.py:23-35). Views and constants never belong
to a kernel."""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel
from kiln.passes.manager import Pass

COMPUTE_KINDS = ("elementwise", "reduction", "matmul")


class OneOpPerKernel(Pass):
    name = "partition"

    def run(self, graph: Graph):
        graph.kernels = []
        for n in graph.nodes:
            k = ops.kind(n.op)
            if k in COMPUTE_KINDS:
                kern = Kernel(f"k{len(graph.kernels)}", k, [n])
                n.attrs["kernel"] = kern.name
                graph.kernels.append(kern)
        return {"kernels": len(graph.kernels)}
