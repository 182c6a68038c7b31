"""Buffer assignment: where every value's elements live.

Kiln's rules (the reference's kiln/passes/buffers.py:35-265; the HIP
lowering reads the result through ``compute_layouts``, ``kernel_inputs`` and
``kernel_outputs``, and the buffer_assign.kir / memory_plan.kir fixtures pin
the annotations):

  * arguments, constants and results live in caller buffers; a value that
    one kernel computes and anything outside that kernel reads gets a
    contiguous buffer of its own (node attribute ``buffer = "output"`` for a
    graph result, ``"arena"`` otherwise); a value used only inside its kernel
    gets none;
  * a view gets no buffer: it is its source read with another offset and
    other strides (annotated ``offset``/``strides``);
  * a ``copy`` kernel is added only where that is impossible: a result that
    no kernel writes (an argument, a constant, a view, a value returned
    twice), a view that strides cannot express (a reshape of a transposed
    value), and the B operand of a matmul whose columns are not contiguous
    (the GEMM family streams B rows along N as 16-byte vectors).

Kernels are renumbered k0, k1, ... in a topological order afterwards (copies
are created out of order).
"""

from __future__ import annotations

from dataclasses import dataclass
from math import prod

from kiln.ir import ops
from kiln.ir.core import Graph, Kernel, Value
from kiln.passes.manager import Pass

ALIGNMENT = 64  # bytes per arena buffer boundary; keeps every buffer 16-byte aligned for vector loads


def contiguous_strides(shape) -> tuple:
    strides = [1] * len(shape)
    for d in range(len(shape) - 2, -1, -1):
        strides[d] = strides[d + 1] * shape[d + 1]
    return tuple(strides)


@dataclass(frozen=True)
class Layout:
    base: tuple       # ("input", i) | ("output", i) | ("const", name) | ("arena", owning Value)
    offset: int       # elements
    shape: tuple
    strides: tuple    # elements

    @property
    def contiguous(self) -> bool:
        return self.strides == contiguous_strides(self.shape)


def _runs(shape, strides):
    """Split (shape, strides) into maximal runs of dims that address one
    evenly strided block, innermost run first: [(elements, innermost stride)].
    A dim continues the run inside it when its stride is the run's extent
    times the run's base stride; a size-1 dim never ends a run."""
    runs = []
    count, base = 1, strides[-1] if strides else 1
    for d in range(len(shape) - 1, -1, -1):
        count *= shape[d]
        continues = d > 0 and (shape[d - 1] == 1 or strides[d - 1] == count * base)
        if not continues:
            runs.append((count, base))
            if d > 0:
                count, base = 1, strides[d - 1]
    return runs


def reshape_strides(shape, strides, new_shape):
    """Strides that show (shape, strides) as ``new_shape`` without moving
    data, or None. PyTorch's rule for views (ATen ``computeStride``), so views
    and copies happen exactly where PyTorch's would: every run of old dims
    must be covered by consecutive new dims whose sizes multiply to the run's
    element count; new size-1 dims fit anywhere."""
    if prod(shape) == 0:
        return contiguous_strides(new_shape)
    out = [0] * len(new_shape)
    d = len(new_shape) - 1
    for count, base in _runs(shape, strides):
        covered = 1
        while d >= 0 and (covered < count or new_shape[d] == 1):
            out[d] = covered * base
            covered *= new_shape[d]
            d -= 1
        if covered != count:
            return None
    return tuple(out) if d < 0 else None


def _transposed(attrs, src, shape):
    return src.offset, tuple(src.strides[axis] for axis in attrs["perm"])


def _sliced(attrs, src, shape):
    dim = attrs["dim"]
    strides = list(src.strides)
    offset = src.offset + attrs["start"] * strides[dim]
    strides[dim] *= attrs.get("step", 1)
    return offset, tuple(strides)


def _expanded(attrs, src, shape):
    new_dims = len(shape) - len(src.shape)
    kept = tuple(0 if (extent == 1 and shape[new_dims + i] != 1) else stride
                 for i, (extent, stride) in enumerate(zip(src.shape, src.strides)))
    return src.offset, (0,) * new_dims + kept


def _reshaped(attrs, src, shape):
    strides = reshape_strides(src.shape, src.strides, shape)
    return None if strides is None else (src.offset, strides)


_VIEW_RULES = {"transpose": _transposed, "slice": _sliced, "expand": _expanded, "reshape": _reshaped}


def view_layout(op, attrs, src: Layout, out_shape):
    """The layout view ``op`` gives ``src``; None when it needs a copy."""
    rule = _VIEW_RULES.get(op)
    if rule is None:
        raise ValueError(op)
    shape = tuple(out_shape)
    found = rule(attrs, src, shape)
    return None if found is None else Layout(src.base, found[0], shape, found[1])


def kernel_outputs(graph: Graph, k: Kernel, users=None):
    """Values computed in ``k`` that a result or another kernel needs, in
    ``k``'s node order."""
    users = graph.users() if users is None else users
    members = set(k.nodes)
    wanted = set(graph.results)
    return [n.out for n in k.nodes
            if n.out in wanted or not members.issuperset(users.get(n.out, ()))]


def kernel_inputs(graph: Graph, k: Kernel):
    """Values ``k`` reads that it does not compute (scalar constants, which
    are inlined, excluded), in first-read order."""
    members = set(k.nodes)
    found = {}
    for n in k.nodes:
        for v in n.inputs:
            outside = v.node is None or v.node not in members
            if outside and not graph.is_scalar_const(v):
                found.setdefault(v, None)
    return list(found)


def compute_layouts(graph: Graph) -> dict:
    """{value: Layout} for every value with storage. Depends only on the
    annotated graph, so the backend recomputes it from parsed IR."""
    result_slot = {}
    for i, r in enumerate(graph.results):
        result_slot.setdefault(r, i)
    layouts = {arg: Layout(("input", i), 0, arg.shape, contiguous_strides(arg.shape))
               for i, arg in enumerate(graph.args)}
    for n in graph.nodes:
        v = n.out
        if n.op == "const":
            if v.type.shape:
                layouts[v] = Layout(("const", n.attrs["name"]), 0, v.shape, contiguous_strides(v.shape))
            continue
        if ops.kind(n.op) == "view":
            src = layouts.get(n.inputs[0])
            seen = None if src is None else view_layout(n.op, n.attrs, src, v.shape)
            if seen is not None:
                layouts[v] = seen
            continue
        where = n.attrs.get("buffer")
        if where is not None:
            base = ("output", result_slot[v]) if where == "output" else ("arena", v)
            layouts[v] = Layout(base, 0, v.shape, contiguous_strides(v.shape))
    return layouts


def _needs_copy(n, layouts):
    """The operand position of ``n`` that must be copied into a contiguous
    buffer first, or None."""
    if ops.kind(n.op) == "view":
        return 0 if n.out not in layouts and n.inputs[0] in layouts else None
    if n.op == "matmul":
        b = n.inputs[1]
        seen = layouts.get(b)
        if seen is not None and b.shape[-1] > 1 and seen.strides[-1] != 1:
            return 1
    return None


class BufferAssignment(Pass):
    name = "buffer-assign"

    @staticmethod
    def _new_copy(graph: Graph, v: Value, at: int) -> Value:
        out = graph.add_node("copy", [v], {}, index=at)
        kernel = Kernel(f"copy{len(graph.kernels)}", "copy", [out.node])
        out.node.attrs["kernel"] = kernel.name
        graph.kernels.append(kernel)
        return out

    def run(self, graph: Graph):
        copies = 0
        # every result written by a kernel of its own into its output slot
        claimed = set()
        for i, r in enumerate(graph.results):
            if r.node is None or "kernel" not in r.node.attrs or r in claimed:
                graph.results[i] = self._new_copy(graph, r, len(graph.nodes))
                copies += 1
            claimed.add(graph.results[i])

        users = graph.users()
        results = set(graph.results)
        for k in graph.kernels:
            for v in kernel_outputs(graph, k, users):
                v.node.attrs["buffer"] = "output" if v in results else "arena"

        # one copy at a time, earliest offending node first, until views and
        # GEMM B operands all have usable layouts
        while True:
            layouts = compute_layouts(graph)
            hit = next(((i, n, p) for i, n in enumerate(graph.nodes)
                        if (p := _needs_copy(n, layouts)) is not None), None)
            if hit is None:
                break
            at, n, operand = hit
            copied = self._new_copy(graph, n.inputs[operand], at)
            copied.node.attrs["buffer"] = "arena"
            n.inputs[operand] = copied
            copies += 1

        for n in graph.nodes:
            if ops.kind(n.op) == "view" and n.out in layouts:
                n.attrs["strides"] = list(layouts[n.out].strides)
                n.attrs["offset"] = layouts[n.out].offset
        order_kernels(graph)
        return {"copies": copies} if copies else None


def order_kernels(graph: Graph):
    """Nodes in topological order, then kernels in topological order of the
    kernel graph (taken by first-node position, each preceded by its not yet
    placed producers, also by first-node position), renamed k0, k1, ...,
    with each kernel's nodes in program order."""
    graph.toposort()
    position = {n: i for i, n in enumerate(graph.nodes)}
    owner = {n: k for k in graph.kernels for n in k.nodes}
    first = {k: position[k.nodes[0]] for k in graph.kernels}

    def producers(k):
        found = set()
        for n in k.nodes:
            for v in n.inputs:
                while v.node is not None and ops.kind(v.node.op) == "view":
                    v = v.node.inputs[0]
                src = owner.get(v.node)
                if src is not None and src is not k:
                    found.add(src)
        return sorted(found, key=first.get)

    ordered, placed = [], set()
    for root in sorted(graph.kernels, key=first.get):
        stack = [(root, iter(producers(root)))]
        if root in placed:
            continue
        placed.add(root)
        while stack:
            k, pending = stack[-1]
            nxt = next((p for p in pending if p not in placed), None)
            if nxt is None:
                ordered.append(k)
                stack.pop()
            else:
                placed.add(nxt)
                stack.append((nxt, iter(producers(nxt))))
    for i, k in enumerate(ordered):
        k.name = f"k{i}"
        k.nodes.sort(key=position.get)
        for n in k.nodes:
            n.attrs["kernel"] = k.name
    graph.kernels = ordered


