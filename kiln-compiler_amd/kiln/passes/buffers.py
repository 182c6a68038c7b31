"""Buffer assignment: where every value lives, as (base, offset, strides).

Contract of the reference's kiln/passes/buffers.py:35-265, which the HIP
lowering consumes (``compute_layouts``, ``kernel_inputs``, ``kernel_outputs``):

  * graph inputs, constants and graph outputs live in caller buffers;
  * a value computed in one kernel and read elsewhere gets a contiguous
    buffer (``buffer = "arena"`` or ``"output"``); values internal to a
    kernel get none;
  * views get no buffer: they are strided reads of their source;
  * a copy kernel is inserted only where a view cannot be expressed with
    strides, or where a matmul's B operand is not contiguous along N (the GEMM
    family streams B rows as 16-byte vectors along N).

The ``strides``/``offset`` annotations on views and the 64-byte alignment are
pinned by the ``buffer_assign.kir`` and ``memory_plan.kir`` fixtures.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import prod

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel, Value
from kiln.passes.manager import Pass

ALIGNMENT = 64  # bytes; also keeps every arena buffer 16-byte aligned for vector loads


@dataclass(frozen=True)
class Layout:
    base: tuple       # ("input", i) | ("output", i) | ("const", name) | ("arena", owner Value)
    offset: int       # elements
    shape: tuple
    strides: tuple    # elements

    @property
    def contiguous(self) -> bool:
        return self.strides == contiguous_strides(self.shape)


def contiguous_strides(shape) -> tuple:
    out, acc = [], 1
    for s in reversed(shape):
        out.append(acc)
        acc *= s
    return tuple(reversed(out))


def reshape_strides(shape, strides, new_shape):
    """Strides that view (shape, strides) as ``new_shape``, or None.

    This is PyTorch's view rule (ATen ``computeStride``): old dims are grouped
    into runs that are contiguous with respect to each other (size-1 dims never
    break a run); a reshape is a view iff every run is covered exactly by a
    run of new dims. Kept identical so views and copies agree with PyTorch.
    """
    if prod(shape) == 0:
        return contiguous_strides(new_shape)
    out = [0] * len(new_shape)
    nd = len(new_shape) - 1
    base = strides[-1] if strides else 1
    chunk = taken = 1
    for od in range(len(shape) - 1, -1, -1):
        chunk *= shape[od]
        if od > 0 and (shape[od - 1] == 1 or strides[od - 1] == chunk * base):
            continue                      # the run continues into the next-outer dim
        while nd >= 0 and (taken < chunk or new_shape[nd] == 1):
            out[nd] = taken * base
            taken *= new_shape[nd]
            nd -= 1
        if taken != chunk:
            return None
        if od > 0:
            base, chunk, taken = strides[od - 1], 1, 1
    return tuple(out) if nd == -1 else None


def view_layout(op, attrs, src: Layout, out_shape):
    """Layout of view ``op`` applied to ``src``; None if it needs a copy."""
    out_shape = tuple(out_shape)
    if op == "transpose":
        return Layout(src.base, src.offset, out_shape, tuple(src.strides[p] for p in attrs["perm"]))
    if op == "slice":
        d = attrs["dim"]
        st = list(src.strides)
        off = src.offset + attrs["start"] * st[d]
        st[d] *= attrs.get("step", 1)
        return Layout(src.base, off, out_shape, tuple(st))
    if op == "expand":
        lead = len(out_shape) - len(src.shape)
        st = [0] * lead + [0 if (s == 1 and out_shape[lead + i] != 1) else t
                           for i, (s, t) in enumerate(zip(src.shape, src.strides))]
        return Layout(src.base, src.offset, out_shape, tuple(st))
    if op == "reshape":
        st = reshape_strides(src.shape, src.strides, out_shape)
        return None if st is None else Layout(src.base, src.offset, out_shape, st)
    raise ValueError(op)


def kernel_outputs(graph: Graph, k: Kernel, users=None):
    """Values computed in ``k`` that a graph result or another kernel needs."""
    users = graph.users() if users is None else users
    inside = set(k.nodes)
    results = set(graph.results)
    return [n.out for n in k.nodes
            if n.out in results or any(u not in inside for u in users.get(n.out, ()))]


def kernel_inputs(graph: Graph, k: Kernel):
    """Values ``k`` reads from outside itself, scalar constants excluded."""
    inside = set(k.nodes)
    seen, out = set(), []
    for n in k.nodes:
        for v in n.inputs:
            if v.node in inside and v.node is not None:
                continue
            if v in seen or graph.is_scalar_const(v):
                continue
            seen.add(v)
            out.append(v)
    return out


def compute_layouts(graph: Graph) -> dict:
    """Layout of every value with storage. A pure function of the annotated
    graph, so the backend can recompute it from parsed IR."""
    lay = {a: Layout(("input", i), 0, a.shape, contiguous_strides(a.shape))
           for i, a in enumerate(graph.args)}
    out_slot = {}
    for i, r in enumerate(graph.results):
        out_slot.setdefault(r, i)
    for n in graph.nodes:
        v = n.out
        if n.op == "const":
            if v.type.rank > 0:
                lay[v] = Layout(("const", n.attrs["name"]), 0, v.shape, contiguous_strides(v.shape))
        elif ops.kind(n.op) == "view":
            src = lay.get(n.inputs[0])
            if src is not None:
                vl = view_layout(n.op, n.attrs, src, v.shape)
                if vl is not None:
                    lay[v] = vl
        elif "buffer" in n.attrs:
            base = ("output", out_slot[v]) if n.attrs["buffer"] == "output" else ("arena", v)
            lay[v] = Layout(base, 0, v.shape, contiguous_strides(v.shape))
    return lay


class BufferAssignment(Pass):
    name = "buffer-assign"

    @staticmethod
    def _copy(graph: Graph, v: Value, before):
        at = len(graph.nodes) if before is None else graph.nodes.index(before)
        c = graph.add_node("copy", [v], {}, index=at)
        k = Kernel(f"copy{len(graph.kernels)}", "copy", [c.node])
        c.node.attrs["kernel"] = k.name
        graph.kernels.append(k)
        return c

    def run(self, graph: Graph):
        copies = 0
        # Every graph result must be written by a kernel into its own output buffer.
        written = set()
        for i, r in enumerate(graph.results):
            if r.node is None or "kernel" not in r.node.attrs or r in written:
                graph.results[i] = self._copy(graph, r, None)
                copies += 1
            written.add(graph.results[i])

        users = graph.users()
        results = set(graph.results)
        for k in graph.kernels:
            for v in kernel_outputs(graph, k, users):
                v.node.attrs["buffer"] = "output" if v in results else "arena"

        # Realise views that strides cannot express, and non-N-contiguous matmul B.
        while True:
            lay = compute_layouts(graph)
            fixed = False
            for n in list(graph.nodes):
                if ops.kind(n.op) == "view" and n.out not in lay and n.inputs[0] in lay:
                    c = self._copy(graph, n.inputs[0], n)
                    c.node.attrs["buffer"] = "arena"
                    n.inputs[0] = c
                    fixed = True
                elif n.op == "matmul":
                    b = n.inputs[1]
                    bl = lay.get(b)
                    if bl is not None and b.shape[-1] > 1 and bl.strides[-1] != 1:
                        c = self._copy(graph, b, n)
                        c.node.attrs["buffer"] = "arena"
                        n.inputs[1] = c
                        fixed = True
                if fixed:
                    copies += 1
                    break
            if not fixed:
                break

        lay = compute_layouts(graph)
        for n in graph.nodes:
            if ops.kind(n.op) == "view" and n.out in lay:
                n.attrs["strides"] = list(lay[n.out].strides)
                n.attrs["offset"] = lay[n.out].offset
        _order_kernels(graph)
        return {"copies": copies} if copies else None


def _order_kernels(graph: Graph):
    """Topological kernel order (copies were appended), renamed k0, k1, ..."""
    graph.toposort()
    pos = {n: i for i, n in enumerate(graph.nodes)}
    owner = {n: k for k in graph.kernels for n in k.nodes}

    def deps(k):
        out = set()
        for n in k.nodes:
            for v in n.inputs:
                src = v
                while src.node is not None and ops.kind(src.node.op) == "view":
                    src = src.node.inputs[0]
                d = owner.get(src.node)
                if d is not None and d is not k:
                    out.add(d)
        return out

    order, done = [], set()

    def visit(k):
        if k in done:
            return
        done.add(k)
        for d in sorted(deps(k), key=lambda d: pos[d.nodes[0]]):
            visit(d)
        order.append(k)

    for k in sorted(graph.kernels, key=lambda k: pos[k.nodes[0]]):
        visit(k)
    for i, k in enumerate(order):
        k.name = f"k{i}"
        for n in k.nodes:
            n.attrs["kernel"] = k.name
        k.nodes.sort(key=pos.get)
    graph.kernels = order
