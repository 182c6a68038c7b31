"""Fusion: partition the compute nodes into kernels.

The partition is the contract between the passes and the HIP kernel
families, so the rules are Kiln's (the reference's kiln/passes/fusion.py:24-234,
pinned by its tests/test_fusion.py:33-132 and the fusion.kir fixture):

  matmul       a contraction plus an elementwise epilogue over its output
               shape -> the GEMM family (the epilogue becomes its tape);
  reduction    innermost-dim reductions and the elementwise ops over the same
               rows -> the row family (LayerNorm, softmax, generic tapes); a
               reduction over other dims is a kernel of its own (K-RED);
  elementwise  a DAG of elementwise ops -> the elementwise family.

The rules, applied to compute nodes in program order:

  1. a matmul always opens a kernel;
  2. any other node may join a kernel that produces one of its operands
     *directly* (through no view), trying matmul kernels first, then row
     kernels, then elementwise ones (operand order within a kind);
  3. it joins only if it fits the kernel (``_fits``), does not read that
     kernel's results through a view (that needs another element's
     finished value: the kernel would depend on itself), and joining creates
     no cycle: no other kernel it reads from may be reachable from the
     candidate;
  4. otherwise it opens a kernel.

Kernels are then numbered k0, k1, ... in a topological order of the kernel
graph that follows program order: kernels are taken by the position of their
first node, each preceded by its not yet numbered producers (again by first
position, recursively).
"""

from __future__ import annotations

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel, Node
from kiln.passes.manager import Pass

_TRY_ORDER = {"matmul": 0, "reduction": 1, "elementwise": 2}


def is_row_reduction(n: Node) -> bool:
    """A keepdim reduction over exactly the innermost dimension."""
    rank = n.inputs[0].type.rank
    return rank >= 1 and list(n.attrs["dims"]) == [rank - 1]


def compute_kind(n: Node):
    kind = ops.kind(n.op)
    return kind if kind in _TRY_ORDER else None


def resolve_view(v):
    """The value whose storage a chain of views reads."""
    while v.node is not None and ops.kind(v.node.op) == "view":
        v = v.node.inputs[0]
    return v


def _row_space(reduction: Node):
    shape = reduction.inputs[0].shape
    return tuple(shape[:-1]), shape[-1]


def _in_row_space(n: Node, space) -> bool:
    """Its result is one value per row, or one per (row, column)."""
    rows, inner = space
    shape = n.out.shape
    return bool(shape) and tuple(shape[:-1]) == rows and shape[-1] in (inner, 1)


class _Kernel:
    """A kernel under construction."""

    __slots__ = ("kind", "nodes", "start", "matmul", "space", "closed", "after")

    def __init__(self, node: Node, start: int):
        self.kind = compute_kind(node)
        self.nodes = [node]
        self.start = start                       # program position of its first node
        self.matmul = node if self.kind == "matmul" else None
        self.space = None                        # (rows, inner) of a row kernel
        self.closed = False                      # a reduction over other dims takes no company
        self.after = set()                       # kernels that read its results
        if self.kind == "reduction":
            if is_row_reduction(node):
                self.space = _row_space(node)
            else:
                self.closed = True


def _fits(n: Node, k: _Kernel, uses) -> bool:
    if k.closed:
        return False
    kind = compute_kind(n)
    if k.kind == "matmul":
        if kind != "elementwise" or n.out.shape != k.matmul.out.shape:
            return False
        # an epilogue may consume the product only if nothing else does
        consumes = any(v.node is k.matmul for v in n.inputs)
        return not consumes or len(uses.get(k.matmul.out, ())) == 1
    if kind == "elementwise":
        return k.kind == "elementwise" or _in_row_space(n, k.space)
    if kind == "reduction" and is_row_reduction(n):
        space = _row_space(n)
        if k.kind == "reduction":
            return space == k.space
        return all(_in_row_space(m, space) for m in k.nodes)   # an elementwise kernel becomes a row kernel
    return False


def _reaches(start: _Kernel, goal: _Kernel) -> bool:
    seen, todo = {start}, [start]
    while todo:
        k = todo.pop()
        if k is goal:
            return True
        for nxt in k.after:
            if nxt not in seen:
                seen.add(nxt)
                todo.append(nxt)
    return False


class Fusion(Pass):
    name = "fusion"

    def run(self, graph: Graph):
        uses = graph.users()
        owner = {}          # node -> _Kernel
        made = []

        def kernel_of(v):
            return owner.get(v.node) if v.node is not None else None

        for position, n in enumerate(graph.nodes):
            kind = compute_kind(n)
            if kind is None:
                continue
            reads = []      # kernels whose results n reads, directly or through views
            via_view = []   # ... of those, the ones read through a view
            direct = []     # kernels producing an operand directly
            for v in n.inputs:
                src = kernel_of(resolve_view(v))
                if src is not None and src not in reads:
                    reads.append(src)
                if v.node is not None and ops.kind(v.node.op) == "view" and src is not None:
                    via_view.append(src)
                d = kernel_of(v)
                if d is not None and d not in direct:
                    direct.append(d)
            home = None
            if kind != "matmul":
                for cand in sorted(direct, key=lambda k: _TRY_ORDER[k.kind]):
                    if (_fits(n, cand, uses) and cand not in via_view
                            and not any(other is not cand and _reaches(cand, other) for other in reads)):
                        home = cand
                        break
            if home is None:
                home = _Kernel(n, position)
                made.append(home)
            else:
                home.nodes.append(n)
                if kind == "reduction" and home.kind == "elementwise":
                    home.kind, home.space = "reduction", _row_space(n)
            owner[n] = home
            for src in reads:
                if src is not home:
                    src.after.add(home)

        graph.kernels = []
        for k in self._numbering(made):
            kernel = Kernel(f"k{len(graph.kernels)}", k.kind, list(k.nodes))
            for m in k.nodes:
                m.attrs["kernel"] = kernel.name
            graph.kernels.append(kernel)
        return {"kernels": len(graph.kernels), "ops": sum(len(k.nodes) for k in graph.kernels)}

    @staticmethod
    def _numbering(made):
        """Kernels in the order described in the module docstring."""
        before = {k: [] for k in made}
        for k in made:
            for nxt in k.after:
                before[nxt].append(k)
        for k in made:
            before[k].sort(key=lambda p: p.start)
        order, placed, on_path = [], set(), set()
        for root in sorted(made, key=lambda k: k.start):
            stack = [(root, iter(before[root]))]
            on_path.add(root)
            while stack:
                k, pending = stack[-1]
                if k in placed:
                    stack.pop()
                    on_path.discard(k)
                    continue
                nxt = next((p for p in pending if p not in placed), None)
                if nxt is not None:
                    if nxt in on_path:
                        raise AssertionError("fusion produced a cycle between kernels")
                    on_path.add(nxt)
                    stack.append((nxt, iter(before[nxt])))
                    continue
                placed.add(k)
                order.append(k)
                on_path.discard(k)
                stack.pop()
        return order
