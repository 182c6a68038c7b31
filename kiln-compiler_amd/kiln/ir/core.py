"""Kiln graph IR: an SSA dataflow graph over statically shaped f32 tensors.

Contract-compatible counterpart of the reference IR (kiln/ir/core.py:28-239):
the same classes, fields and query/mutation methods, because every pass and
the HIP backend's lowering consume exactly these objects.

  * Every node produces one value; values are immutable and carry no layout.
  * Layout (strides, aliasing) is decided late, by buffer assignment.
  * Passes annotate nodes with attributes (``kernel``, ``buffer``, ``offset``,
    ``strides``), so one printer/parser covers every stage.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import prod

import numpy as np

ELEMENT_BYTES = 4  # every Kiln tensor is f32


@dataclass(frozen=True)
class TensorType:
    """Static shape + element type (reference: kiln/ir/core.py:28-46)."""

    shape: tuple
    dtype: str = "f32"

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        return prod(self.shape)

    @property
    def nbytes(self) -> int:
        return self.numel * ELEMENT_BYTES

    def __str__(self):
        return "%s[%s]" % (self.dtype, ", ".join(str(d) for d in self.shape))


class Value:
    """An SSA value: a graph argument (``node is None``) or a node's result."""

    __slots__ = ("type", "node", "name")

    def __init__(self, type: TensorType, node=None, name=None):
        self.type = type
        self.node = node
        self.name = name

    @property
    def shape(self):
        return self.type.shape

    @property
    def is_arg(self) -> bool:
        return self.node is None

    def __repr__(self):
        src = "arg" if self.node is None else self.node.op
        return f"<Value {self.name or '?'}: {self.type} from {src}>"


class Node:
    """One operation; owns its single result ``out``."""

    __slots__ = ("op", "inputs", "attrs", "out")

    def __init__(self, op: str, inputs, attrs: dict, out_type: TensorType):
        self.op = op
        self.inputs = list(inputs)
        self.attrs = dict(attrs)
        self.out = Value(out_type, self)

    def __repr__(self):
        return f"<Node {self.op} -> {self.out.type}>"


@dataclass(eq=False)
class Kernel:
    """A fusion group compiled into one device program (kind: elementwise |
    reduction | matmul | copy)."""

    name: str
    kind: str
    nodes: list = field(default_factory=list)
    attrs: dict = field(default_factory=dict)


class Graph:
    """The whole program: arguments, nodes in program order, results,
    kernel partition and constant data (reference: kiln/ir/core.py:95-214)."""

    def __init__(self, name: str = "forward"):
        self.name = name
        self.args: list = []
        self.arg_attrs: list = []
        self.nodes: list = []
        self.results: list = []
        self.attrs: dict = {}
        self.kernels: list = []
        self.constants: dict = {}

    # construction ---------------------------------------------------------

    def add_arg(self, type: TensorType, name: str, **attrs) -> Value:
        v = Value(type, None, name)
        self.args.append(v)
        self.arg_attrs.append(dict(attrs))
        return v

    def add_node(self, op, inputs, attrs=None, out_type=None, index=None) -> Value:
        """Append (or insert at ``index``) a node; infers the type if not given."""
        from kiln.ir.ops import infer_type

        attrs = dict(attrs or {})
        if out_type is None:
            out_type = infer_type(op, [v.type for v in inputs], attrs)
        node = Node(op, inputs, attrs, out_type)
        if index is None:
            self.nodes.append(node)
        else:
            self.nodes.insert(index, node)
        return node.out

    def constant(self, array, name: str, index=None) -> Value:
        """A named tensor constant; its data goes to ``self.constants`` under a
        unique name (``name``, ``name_1``, ...)."""
        data = np.ascontiguousarray(array, dtype=np.float32)
        unique, n = name, 0
        while unique in self.constants:
            n += 1
            unique = f"{name}_{n}"
        self.constants[unique] = data
        return self.add_node("const", [], {"name": unique}, TensorType(tuple(data.shape)), index)

    def scalar(self, value: float, index=None) -> Value:
        return self.add_node("const", [], {"value": float(value)}, TensorType(()), index)

    # queries ----------------------------------------------------------------

    def users(self) -> dict:
        """Value -> nodes that read it, in program order."""
        out: dict = {}
        for n in self.nodes:
            for v in n.inputs:
                out.setdefault(v, []).append(n)
        return out

    def is_const(self, v: Value) -> bool:
        return v.node is not None and v.node.op == "const"

    def is_scalar_const(self, v: Value) -> bool:
        return self.is_const(v) and v.type.rank == 0

    def const_data(self, v: Value):
        node = v.node
        assert node is not None and node.op == "const", v
        if "value" in node.attrs:
            return np.asarray(node.attrs["value"], dtype=np.float32)
        return self.constants[node.attrs["name"]]

    def kernel_of(self, node: Node):
        name = node.attrs.get("kernel")
        return next((k for k in self.kernels if k.name == name), None)

    # mutation ----------------------------------------------------------------

    def replace_all_uses(self, old: Value, new: Value):
        for n in self.nodes:
            if any(v is old for v in n.inputs):
                n.inputs = [new if v is old else v for v in n.inputs]
        self.results = [new if v is old else v for v in self.results]

    def remove_dead(self) -> int:
        """Drop nodes that no result depends on, and constant data nobody names.
        Returns the number of nodes removed."""
        needed = set(self.results)
        keep = []
        for n in reversed(self.nodes):
            if n.out in needed:
                keep.append(n)
                needed.update(n.inputs)
        removed = len(self.nodes) - len(keep)
        keep.reverse()
        self.nodes = keep
        names = {n.attrs["name"] for n in keep if n.op == "const" and "name" in n.attrs}
        names.update(a["param"] for a in self.arg_attrs if "param" in a)
        self.constants = {k: d for k, d in self.constants.items() if k in names}
        return removed

    def toposort(self):
        """Stable topological re-ordering of ``nodes`` (iterative DFS)."""
        members = set(self.nodes)
        done, order = set(), []
        for root in self.nodes:
            if root in done:
                continue
            stack = [(root, iter(root.inputs))]
            done.add(root)
            while stack:
                node, it = stack[-1]
                pushed = False
                for v in it:
                    p = v.node
                    if p is not None and p in members and p not in done:
                        done.add(p)
                        stack.append((p, iter(p.inputs)))
                        pushed = True
                        break
                if not pushed:
                    stack.pop()
                    order.append(node)
        self.nodes = order

    def __str__(self):
        from kiln.ir.printer import print_graph

        return print_graph(self)


def verify(graph: Graph):
    """SSA dominance, known ops, const data present, types equal inference
    (reference: kiln/ir/core.py:217-239). Raises ValueError."""
    from kiln.ir.ops import OPS, infer_type

    defined = set(graph.args)
    for n in graph.nodes:
        if n.op not in OPS:
            raise ValueError(f"unknown op '{n.op}'")
        for v in n.inputs:
            if v not in defined:
                raise ValueError(f"{n.op}: operand used before definition: {v}")
        if n.op == "const":
            if "value" in n.attrs:
                if n.out.type.rank != 0:
                    raise ValueError("const with 'value' must be a scalar (f32[])")
            elif n.attrs.get("name") not in graph.constants:
                raise ValueError(f"const refers to missing data '{n.attrs.get('name')}'")
        else:
            want = infer_type(n.op, [v.type for v in n.inputs], n.attrs)
            if want != n.out.type:
                raise ValueError(f"{n.op}: type {n.out.type} does not match inferred {want}")
        defined.add(n.out)
    for v in graph.results:
        if v not in defined:
            raise ValueError(f"result {v} is not defined in the graph")
