"""Clean-up passes: Canonicalize, CSE and DCE.

The rewrites are Kiln's (the reference's kiln/passes/simplify.py:19-97; the
FileCheck fixture tests/lit/canonicalize.kir pins them):

  * a view that changes nothing (reshape / expand / slice to the operand's
    own shape, transpose by the identity permutation) is its operand;
  * reshape of a reshape is one reshape; transpose of a transpose is one
    transpose by the composed permutation;
  * x + 0, x - 0, x * 1, x / 1 (scalar constant on the right) and 0 + x,
    1 * x (on the left) are x, as long as the result has x's shape (a
    broadcast against a bigger constant is kept).

Canonicalize walks the nodes once, front to back. Operands are always
already canonical when a node is reached (they come earlier), so a node is
rewritten until no rule applies and the walk never has to restart: a rule
that builds a replacement node puts it in the node's place and the walk
continues from it.
"""

from __future__ import annotations

from kiln.ir.core import Graph, Node
from kiln.passes.manager import Pass

_IDENTITY_ON_SAME_SHAPE = ("reshape", "expand", "slice")
_NEUTRAL = {"add": (0.0, True), "sub": (0.0, False), "mul": (1.0, True), "div": (1.0, False)}


def _scalar_equals(g: Graph, v, number: float) -> bool:
    return g.is_scalar_const(v) and float(g.const_data(v)) == number


def _fold_view(g: Graph, node: Node):
    """Rules on views. Returns an equivalent Value, a replacement (op,
    operand, attrs) triple, or None."""
    op, x = node.op, node.inputs[0]
    if op in _IDENTITY_ON_SAME_SHAPE and x.shape == node.out.shape:
        return x
    if op == "transpose":
        perm = list(node.attrs["perm"])
        if perm == sorted(perm):
            return x
        inner = x.node
        if inner is not None and inner.op == "transpose":
            first = inner.attrs["perm"]
            return ("transpose", inner.inputs[0], {"perm": [first[p] for p in perm]})
    if op == "reshape" and x.node is not None and x.node.op == "reshape":
        return ("reshape", x.node.inputs[0], {"shape": list(node.out.shape)})
    return None


def _fold_arith(g: Graph, node: Node):
    neutral, commutes = _NEUTRAL[node.op]
    lhs, rhs = node.inputs
    if _scalar_equals(g, rhs, neutral) and lhs.shape == node.out.shape:
        return lhs
    if commutes and _scalar_equals(g, lhs, neutral) and rhs.shape == node.out.shape:
        return rhs
    return None


class Canonicalize(Pass):
    name = "canonicalize"

    def simplify(self, g: Graph, node: Node):
        if node.op in ("reshape", "expand", "slice", "transpose"):
            return _fold_view(g, node)
        if node.op in _NEUTRAL:
            return _fold_arith(g, node)
        return None

    def run(self, g: Graph):
        rewrites, i = 0, 0
        while i < len(g.nodes):
            node = g.nodes[i]
            found = self.simplify(g, node)
            if found is None or found is node.out:
                i += 1
                continue
            del g.nodes[i]
            if isinstance(found, tuple):
                op, operand, attrs = found
                found = g.add_node(op, [operand], attrs, index=i)   # revisited at position i
            g.replace_all_uses(node.out, found)
            rewrites += 1
        return {"rewrites": rewrites} if rewrites else None


def _hashable(obj):
    if isinstance(obj, dict):
        return tuple(sorted((k, _hashable(v)) for k, v in obj.items()))
    if isinstance(obj, (list, tuple)):
        return ("[", *map(_hashable, obj))
    return obj


class CSE(Pass):
    """Nodes with the same op, operands (by identity), attributes and type
    compute the same value: keep the first, forward the rest to it."""

    name = "cse"

    def run(self, g: Graph):
        first_of, merged, kept = {}, 0, []
        for node in g.nodes:
            key = (node.op, tuple(id(v) for v in node.inputs), _hashable(node.attrs), node.out.type)
            twin = first_of.setdefault(key, node.out)
            if twin is node.out:
                kept.append(node)
                continue
            g.replace_all_uses(node.out, twin)
            merged += 1
        g.nodes = kept
        return {"removed": merged} if merged else None


class DCE(Pass):
    name = "dce"

    def run(self, g: Graph):
        removed = g.remove_dead()
        return {"removed": removed} if removed else None
