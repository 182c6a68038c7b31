"""Cleanup passes: canonicalisation, CSE and DCE.

Same rewrites as the reference (kiln/passes/simplify.py:19-97), which the
FileCheck fixture ``canonicalize.kir`` pins:
  * identity views (reshape/expand to the same shape, identity permutation,
    full slice) are replaced by their operand;
  * reshape(reshape(x)) -> reshape(x); transpose(transpose(x)) -> one
    transpose with the composed permutation;
  * x*1, x/1, x+0, x-0, 1*x, 0+x with a scalar constant -> x (only when the
    result shape equals x's, so no broadcast is lost).
"""

from __future__ import annotations

from kiln.ir.core import Graph
from kiln.passes.manager import Pass


class Canonicalize(Pass):
    name = "canonicalize"

    @staticmethod
    def _is_neutral(g: Graph, v, neutral: float) -> bool:
        return g.is_scalar_const(v) and float(g.const_data(v)) == neutral

    def rewrite(self, g: Graph, n):
        """Return a value equivalent to ``n.out`` or None."""
        op, ins = n.op, n.inputs
        if op in ("reshape", "expand", "slice") and n.out.shape == ins[0].shape:
            return ins[0]
        if op == "transpose" and list(n.attrs["perm"]) == list(range(len(n.attrs["perm"]))):
            return ins[0]
        src = ins[0].node if ins else None
        if src is not None and src.op == op == "reshape":
            return g.add_node("reshape", [src.inputs[0]], {"shape": list(n.out.shape)},
                              index=g.nodes.index(n))
        if src is not None and src.op == op == "transpose":
            inner, outer = src.attrs["perm"], n.attrs["perm"]
            return g.add_node("transpose", [src.inputs[0]], {"perm": [inner[p] for p in outer]},
                              index=g.nodes.index(n))
        if op in ("add", "sub", "mul", "div"):
            a, b = ins
            neutral = 0.0 if op in ("add", "sub") else 1.0
            if self._is_neutral(g, b, neutral) and a.shape == n.out.shape:
                return a
            if op in ("add", "mul") and self._is_neutral(g, a, neutral) and b.shape == n.out.shape:
                return b
        return None

    def run(self, g: Graph):
        count = 0
        progress = True
        while progress:
            progress = False
            for n in list(g.nodes):
                if n not in g.nodes:
                    continue
                new = self.rewrite(g, n)
                if new is None or new is n.out:
                    continue
                g.replace_all_uses(n.out, new)
                g.nodes.remove(n)
                count += 1
                progress = True
        return {"rewrites": count} if count else None


class CSE(Pass):
    """Merge nodes with the same op, operands, attributes and type."""

    name = "cse"

    def run(self, g: Graph):
        table, removed = {}, 0
        for n in list(g.nodes):
            key = (n.op, tuple(map(id, n.inputs)), repr(sorted(n.attrs.items())), n.out.type)
            prior = table.get(key)
            if prior is None:
                table[key] = n.out
                continue
            g.replace_all_uses(n.out, prior)
            g.nodes.remove(n)
            removed += 1
        return {"removed": removed} if removed else None


class DCE(Pass):
    name = "dce"

    def run(self, g: Graph):
        removed = g.remove_dead()
        return {"removed": removed} if removed else None
