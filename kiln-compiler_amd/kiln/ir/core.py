"""The graph IR this build compiles: SSA values over static-shape f32 tensors.

A ``Graph`` is an ordered list of ``Node``s. Every node yields exactly one
``Value``; graph arguments are Values without a node. Nothing in the IR says
how a tensor is laid out: buffer assignment later records ``buffer``,
``offset`` and ``strides`` as node attributes, and fusion records ``kernel``
(the name of the ``Kernel`` the node belongs to), so one text form (printer /
parser) shows the graph at every stage.

The interface is Kiln's (class, field and method names of the reference's
kiln/ir/core.py:28-239), because the passes, the text form and the HIP
lowering are all written against it; the implementation is this build's own.
"""

from __future__ import annotations

from collections import defaultdict
from dataclasses import dataclass, field
from math import prod
from typing import NamedTuple

import numpy as np


class TensorType(NamedTuple):
    """Static shape and element type (only "f32" is produced)."""

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
        return 4 * self.numel

    def __str__(self) -> str:
        return self.dtype + "[" + ", ".join(map(str, self.shape)) + "]"


class Value:
    """An SSA value. ``node`` is the producer (None for a graph argument);
    ``name`` is kept for arguments and used as a printing hint."""

    __slots__ = ("type", "node", "name")

    def __init__(self, type: TensorType, node: "Node | None" = None, name: str | None = None):
        self.type, self.node, self.name = type, node, name

    shape = property(lambda self: self.type.shape)
    is_arg = property(lambda self: self.node is None)

    def __repr__(self) -> str:
        made_by = "arg" if self.node is None else self.node.op
        return f"<Value {self.name or '?'}: {self.type} from {made_by}>"


class Node:
    """One operation; ``out`` is the Value it defines."""

    __slots__ = ("op", "inputs", "attrs", "out")

    def __init__(self, op: str, inputs, attrs: dict, out_type: TensorType):
        self.op = op
        self.inputs = list(inputs)
        self.attrs = dict(attrs)
        self.out = Value(out_type, self)

    def __repr__(self) -> str:
        return f"<Node {self.op} -> {self.out.type}>"


@dataclass(eq=False)
class Kernel:
    """A fusion group, compiled as one device program. ``kind`` is
    elementwise, reduction, matmul or copy."""

    name: str
    kind: str
    nodes: list = field(default_factory=list)
    attrs: dict = field(default_factory=dict)


class Graph:
    """Arguments (``args`` with per-argument ``arg_attrs``; ``param = name``
    marks a weight whose data is in ``constants``), ``nodes`` in program
    order, ``results``, graph ``attrs`` (``arena_bytes`` after planning), the
    ``kernels`` partition and the named constant arrays."""

    def __init__(self, name: str = "forward"):
        self.name = name
        self.args = []
        self.arg_attrs = []
        self.nodes = []
        self.results = []
        self.attrs = {}
        self.kernels = []
        self.constants = {}

    # -- building -------------------------------------------------------------------

    def add_arg(self, type: TensorType, name: str, **attrs) -> Value:
        arg = Value(type, None, name)
        self.args.append(arg)
        self.arg_attrs.append(attrs)
        return arg

    def add_node(self, op: str, inputs, attrs=None, out_type=None, index=None) -> Value:
        """New node defining a new value; the type is inferred from the op
        table unless given. ``index`` inserts it before that position."""
        inputs = list(inputs)
        attrs = {} if attrs is None else dict(attrs)
        if out_type is None:
            from kiln.ir.ops import infer_type

            out_type = infer_type(op, [v.type for v in inputs], attrs)
        node = Node(op, inputs, attrs, out_type)
        self.nodes.insert(len(self.nodes) if index is None else index, node)
        return node.out

    def constant(self, array, name: str, index=None) -> Value:
        """A tensor constant. Its data is stored under ``name``, or under
        ``name_<k>`` with the smallest k that is still free."""
        data = np.ascontiguousarray(array, dtype=np.float32)
        key, k = name, 0
        while key in self.constants:
            k += 1
            key = f"{name}_{k}"
        self.constants[key] = data
        return self.add_node("const", [], {"name": key}, TensorType(tuple(data.shape)), index)

    def scalar(self, value: float, index=None) -> Value:
        return self.add_node("const", [], {"value": float(value)}, TensorType(()), index)

    # -- questions ------------------------------------------------------------------

    def users(self) -> dict:
        """{value: [nodes reading it, in program order]}; a node that reads a
        value twice is listed twice."""
        readers = defaultdict(list)
        for node in self.nodes:
            for v in node.inputs:
                readers[v].append(node)
        return dict(readers)

    def is_const(self, v: Value) -> bool:
        return v.node is not None and v.node.op == "const"

    def is_scalar_const(self, v: Value) -> bool:
        return self.is_const(v) and not v.type.shape

    def const_data(self, v: Value) -> np.ndarray:
        if not self.is_const(v):
            raise ValueError(f"{v} is not a constant")
        attrs = v.node.attrs
        if "value" in attrs:
            return np.asarray(attrs["value"], dtype=np.float32)
        return self.constants[attrs["name"]]

    def kernel_of(self, node: Node):
        wanted = node.attrs.get("kernel")
        for kernel in self.kernels:
            if kernel.name == wanted:
                return kernel
        return None

    # -- rewriting ------------------------------------------------------------------

    def replace_all_uses(self, old: Value, new: Value):
        for node in self.nodes:
            if old in node.inputs:
                node.inputs = [new if v is old else v for v in node.inputs]
        if old in self.results:
            self.results = [new if v is old else v for v in self.results]

    def remove_dead(self) -> int:
        """Delete nodes no result depends on, then constant arrays that no
        const node or param argument names. Returns the nodes deleted."""
        live = set()
        pending = [v for v in self.results if v.node is not None]
        while pending:
            node = pending.pop().node
            if node in live:
                continue
            live.add(node)
            pending.extend(v for v in node.inputs if v.node is not None and v.node not in live)
        before = len(self.nodes)
        self.nodes = [n for n in self.nodes if n in live]
        named = {n.attrs["name"] for n in self.nodes if n.op == "const" and "name" in n.attrs}
        named.update(a["param"] for a in self.arg_attrs if "param" in a)
        for key in [k for k in self.constants if k not in named]:
            del self.constants[key]
        return before - len(self.nodes)

    def toposort(self):
        """Order nodes so every operand's producer comes first. Stable: a node
        keeps its place unless a producer listed after it must move ahead, in
        which case that producer (and its own late producers, recursively, in
        operand order) is emitted right before the first node that needs it."""
        position = {n: i for i, n in enumerate(self.nodes)}
        placed, order = set(), []
        for root in self.nodes:
            # explicit stack of (node, index of the next operand to look at)
            stack = [[root, 0]]
            while stack:
                frame = stack[-1]
                node, i = frame
                if node in placed:
                    stack.pop()
                    continue
                if i < len(node.inputs):
                    frame[1] += 1
                    producer = node.inputs[i].node
                    if producer is not None and producer in position and producer not in placed:
                        stack.append([producer, 0])
                    continue
                placed.add(node)
                order.append(node)
                stack.pop()
        self.nodes = order

    def __str__(self) -> str:
        from kiln.ir.printer import print_graph

        return print_graph(self)


def verify(graph: Graph):
    """Raise ValueError unless the graph is well formed: every op is known,
    every operand is defined before its use, const nodes have their data,
    node types agree with the op table and every result is defined."""
    from kiln.ir.ops import OPS, infer_type

    seen = set(graph.args)
    for node in graph.nodes:
        if node.op not in OPS:
            raise ValueError(f"unknown op '{node.op}'")
        missing = [v for v in node.inputs if v not in seen]
        if missing:
            raise ValueError(f"{node.op}: operand used before definition: {missing[0]}")
        if node.op != "const":
            inferred = infer_type(node.op, [v.type for v in node.inputs], node.attrs)
            if inferred != node.out.type:
                raise ValueError(f"{node.op}: type {node.out.type} does not match inferred {inferred}")
        elif "value" in node.attrs:
            if node.out.type.shape:
                raise ValueError("const with 'value' must be a scalar (f32[])")
        elif node.attrs.get("name") not in graph.constants:
            raise ValueError(f"const refers to missing data '{node.attrs.get('name')}'")
        seen.add(node.out)
    for v in graph.results:
        if v not in seen:
            raise ValueError(f"result {v} is not defined in the graph")
