"""Operator fusion: partition compute nodes into kernels.

The partition is the contract between the compiler and the HIP kernel
families, so it follows the reference's greedy rules exactly
(kiln/passes/fusion.py:24-234; pinned by tests/test_fusion.py:33-132 and the
``fusion.kir`` fixture):

  matmul       a contraction plus an elementwise epilogue over its output
               shape -> the MFMA GEMM family with an epilogue tape;
  reduction    innermost-dim reductions plus elementwise ops over the same
               rows -> the row family (LayerNorm, softmax, generic tapes);
               a reduction over other dims stays alone -> the K-RED family;
  elementwise  a DAG of elementwise ops -> the vectorised elementwise family.

Nodes are visited in program order. A node may join a *direct* producer's
group (views end groups) if the kinds are compatible, the join creates no
cycle between groups, and the node does not read that group's own results
through a view. A matmul result with other users takes no epilogue.
"""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel, Node
from kiln.passes.manager import Pass

_RANK = {"matmul": 0, "reduction": 1, "elementwise": 2}


def is_row_reduction(n: Node) -> bool:
    """keepdim reduction over exactly the innermost dim."""
    r = n.inputs[0].type.rank
    return r >= 1 and list(n.attrs["dims"]) == [r - 1]


def compute_kind(n: Node):
    k = ops.kind(n.op)
    return k if k in _RANK else None


def resolve_view(v):
    """The value that owns the storage a chain of views reads."""
    while v.node is not None and ops.kind(v.node.op) == "view":
        v = v.node.inputs[0]
    return v


class _Group:
    __slots__ = ("kind", "nodes", "anchor", "rows", "inner", "fusible", "first")

    def __init__(self, kind, node, first):
        self.kind = kind
        self.nodes = [node]
        self.first = first
        self.anchor = node if kind == "matmul" else None
        self.rows = self.inner = None
        self.fusible = True
        if kind == "reduction":
            if is_row_reduction(node):
                self.set_rows(node)
            else:
                self.fusible = False

    def set_rows(self, reduction: Node):
        shape = reduction.inputs[0].shape
        self.rows, self.inner = tuple(shape[:-1]), shape[-1]


def _row_shaped(n: Node, rows, inner) -> bool:
    s = n.out.shape
    return len(s) >= 1 and tuple(s[:-1]) == tuple(rows) and s[-1] in (inner, 1)


class Fusion(Pass):
    name = "fusion"

    @staticmethod
    def _reaches(src, dst, succ) -> bool:
        todo, seen = [src], {src}
        while todo:
            g = todo.pop()
            if g is dst:
                return True
            for s in succ.get(g, ()):
                if s not in seen:
                    seen.add(s)
                    todo.append(s)
        return False

    @staticmethod
    def _compatible(n: Node, g: _Group, group_of, users) -> bool:
        if not g.fusible:
            return False
        kind = compute_kind(n)
        if g.kind == "matmul":
            if kind != "elementwise" or n.out.shape != g.anchor.out.shape:
                return False
            reads_anchor = any(v.node is g.anchor for v in n.inputs)
            return not (reads_anchor and len(users.get(g.anchor.out, ())) != 1)
        if kind == "elementwise":
            return True if g.kind == "elementwise" else _row_shaped(n, g.rows, g.inner)
        if kind == "reduction" and is_row_reduction(n):
            shape = n.inputs[0].shape
            rows, inner = tuple(shape[:-1]), shape[-1]
            if g.kind == "reduction":
                return (rows, inner) == (g.rows, g.inner)
            return all(_row_shaped(m, rows, inner) for m in g.nodes)
        return False

    def run(self, graph: Graph):
        users = graph.users()
        group_of: dict = {}
        groups: list = []
        succ: dict = {}
        position = {n: i for i, n in enumerate(graph.nodes)}

        def producers(n, via_view_only=False):
            found = []
            for v in n.inputs:
                through_view = v.node is not None and ops.kind(v.node.op) == "view"
                if via_view_only and not through_view:
                    continue
                src = resolve_view(v).node
                g = group_of.get(src) if src is not None else None
                if g is not None and g not in found:
                    found.append(g)
            return found

        for n in graph.nodes:
            kind = compute_kind(n)
            if kind is None:
                continue
            target = None
            if kind != "matmul":
                direct = []
                for v in n.inputs:
                    g = group_of.get(v.node) if v.node is not None else None
                    if g is not None and g not in direct:
                        direct.append(g)
                direct.sort(key=lambda g: _RANK[g.kind])
                everyone = producers(n)
                via_view = producers(n, via_view_only=True)
                for g in direct:
                    if not self._compatible(n, g, group_of, users):
                        continue
                    if g in via_view:
                        continue
                    if any(h is not g and self._reaches(g, h, succ) for h in everyone):
                        continue
                    target = g
                    break
            if target is None:
                target = _Group(kind, n, position[n])
                groups.append(target)
            else:
                target.nodes.append(n)
                if kind == "reduction" and target.kind == "elementwise":
                    target.kind = "reduction"
                    target.set_rows(n)
            group_of[n] = target
            for h in producers(n):
                if h is not target:
                    succ.setdefault(h, set()).add(target)

        preds = {g: [] for g in groups}
        for h, targets in succ.items():
            for t in targets:
                preds[t].append(h)
        order, state = [], {}

        def visit(g):
            st = state.get(g)
            if st == "done":
                return
            if st == "open":
                raise AssertionError("fusion produced a cycle between kernels")
            state[g] = "open"
            for p in sorted(preds[g], key=lambda x: x.first):
                visit(p)
            state[g] = "done"
            order.append(g)

        for g in sorted(groups, key=lambda x: x.first):
            visit(g)

        graph.kernels = []
        for i, g in enumerate(order):
            k = Kernel(f"k{i}", g.kind, list(g.nodes))
            for m in g.nodes:
                m.attrs["kernel"] = k.name
            graph.kernels.append(k)
        return {"kernels": len(graph.kernels), "ops": sum(len(k.nodes) for k in graph.kernels)}
