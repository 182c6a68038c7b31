"""Weight freezing and constant folding (reference: kiln/passes/freeze.py:25-75).

Freezing turns ``param`` arguments into named constants. Folding then
evaluates every node whose operands are all constants. For ``nn.Linear`` that
folds ``W.t()`` into a constant ``"<name>.transpose"`` stored as [K, N] with N
contiguous: the B layout the HIP GEMM streams without a transposing load (the
frozen weight is prepacked once at compile time).

A fold that would *grow* data (e.g. expanding a scalar to a matrix) is refused:
a broadcast is a free stride-0 view, materialising it costs HBM bandwidth.
"""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph
from kiln.passes.manager import Pass


class FreezeParameters(Pass):
    name = "freeze"

    def run(self, g: Graph):
        frozen = 0
        args, attrs = [], []
        for a, at in zip(g.args, g.arg_attrs):
            if "param" not in at:
                args.append(a)
                attrs.append(at)
                continue
            c = g.add_node("const", [], {"name": at["param"]}, a.type, index=frozen)
            g.replace_all_uses(a, c)
            frozen += 1
        g.args, g.arg_attrs = args, attrs
        return {"frozen": frozen} if frozen else None


class ConstantFold(Pass):
    name = "const-fold"

    def run(self, g: Graph):
        folded = nbytes = 0
        for n in list(g.nodes):
            if n.op == "const" or not n.inputs or not all(g.is_const(v) for v in n.inputs):
                continue
            if n.out.type.numel > max(max(v.type.numel for v in n.inputs), 1):
                continue
            data = ops.evaluate(n.op, [g.const_data(v) for v in n.inputs], n.attrs)
            at = g.nodes.index(n)
            if n.out.type.rank == 0:
                new = g.scalar(float(data), index=at)
            else:
                stem = next((v.node.attrs["name"] for v in n.inputs if "name" in v.node.attrs), "folded")
                new = g.constant(data, f"{stem}.{n.op}", index=at)
                nbytes += data.nbytes
            g.replace_all_uses(n.out, new)
            g.nodes.remove(n)
            folded += 1
        g.remove_dead()
        return {"folded": folded, "bytes": nbytes} if folded else None
