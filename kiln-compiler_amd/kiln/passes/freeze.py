"""Freezing and constant folding (Kiln's passes, the reference's
kiln/passes/freeze.py:25-75).

``FreezeParameters`` turns every ``param`` argument into a named ``const``
node (placed at the top of the graph, in argument order) and drops the
argument. ``ConstantFold`` then evaluates, front to back, every node whose
operands are all constants. A tensor result becomes the constant
``"<first named operand>.<op>"`` (so ``nn.Linear``'s ``W.t()`` becomes
``"fc.weight.transpose"``, stored [K, N] with N contiguous: the B layout the
HIP GEMM streams), a scalar result a scalar const. A fold whose result would
hold more elements than its largest operand is skipped: a broadcast costs
nothing as a stride-0 view and HBM bandwidth once materialised.
"""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph
from kiln.passes.manager import Pass


class FreezeParameters(Pass):
    name = "freeze"

    def run(self, g: Graph):
        keep = [(a, attrs) for a, attrs in zip(g.args, g.arg_attrs) if "param" not in attrs]
        frozen = [(a, attrs["param"]) for a, attrs in zip(g.args, g.arg_attrs) if "param" in attrs]
        for position, (arg, pname) in enumerate(frozen):
            const = g.add_node("const", [], {"name": pname}, arg.type, index=position)
            g.replace_all_uses(arg, const)
        g.args = [a for a, _ in keep]
        g.arg_attrs = [attrs for _, attrs in keep]
        return {"frozen": len(frozen)} if frozen else None


class ConstantFold(Pass):
    name = "const-fold"

    @staticmethod
    def _foldable(g: Graph, node) -> bool:
        if node.op == "const" or not node.inputs:
            return False
        if not all(g.is_const(v) for v in node.inputs):
            return False
        largest = max(1, *(v.type.numel for v in node.inputs))
        return node.out.type.numel <= largest

    def run(self, g: Graph):
        folded, new_bytes, i = 0, 0, 0
        while i < len(g.nodes):
            node = g.nodes[i]
            if not self._foldable(g, node):
                i += 1
                continue
            data = ops.evaluate(node.op, [g.const_data(v) for v in node.inputs], node.attrs)
            del g.nodes[i]
            if node.out.type.rank == 0:
                value = g.scalar(float(data), index=i)
            else:
                stems = [v.node.attrs["name"] for v in node.inputs if "name" in v.node.attrs]
                value = g.constant(data, f"{stems[0] if stems else 'folded'}.{node.op}", index=i)
                new_bytes += data.nbytes
            g.replace_all_uses(node.out, value)
            folded += 1
            i += 1
        g.remove_dead()
        return {"folded": folded, "bytes": new_bytes} if folded else None
