"""``fusion=False``: every compute node is its own kernel (Kiln's ablation
baseline, the reference's kiln/passes/partition.py:23-35). Views and
constants belong to no kernel; kernels are numbered k0, k1, ... in program
order."""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel
from kiln.passes.manager import Pass

COMPUTE_KINDS = ("elementwise", "reduction", "matmul")


class OneOpPerKernel(Pass):
    name = "partition"

    def run(self, graph: Graph):
        compute = [n for n in graph.nodes if ops.kind(n.op) in COMPUTE_KINDS]
        graph.kernels = [Kernel(f"k{i}", ops.kind(n.op), [n]) for i, n in enumerate(compute)]
        for node, kernel in zip(compute, graph.kernels):
            node.attrs["kernel"] = kernel.name
        return {"kernels": len(graph.kernels)}
