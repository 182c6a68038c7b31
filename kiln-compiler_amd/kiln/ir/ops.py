"""Op table of the Kiln IR: kind, shape inference and NumPy semantics.

Contract-compatible with the reference op set (kiln/ir/ops.py:48-188): the
same op names, attributes, kinds and result shapes. The NumPy semantics are
used by the constant folder at compile time and by ``interpret`` (public API,
used for pass-level tests); the HIP backend never calls them at run time.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from math import prod
from typing import Callable

import numpy as np

from kiln.ir.core import Graph, TensorType


@dataclass(frozen=True)
class OpDef:
    kind: str            # elementwise | reduction | matmul | view | const
    infer: Callable      # (input shapes, attrs) -> output shape (or None)
    ref: Callable        # (numpy inputs, attrs) -> numpy array
    arity: int | None = None


OPS: dict = {}


def _def(name, kind, infer, ref, arity):
    OPS[name] = OpDef(kind, infer, ref, arity)


def broadcast_shapes(*shapes):
    return tuple(np.broadcast_shapes(*shapes))


# elementwise -------------------------------------------------------------------

_erf64 = np.frompyfunc(math.erf, 1, 1)


def _erf(x):
    return _erf64(np.asarray(x, dtype=np.float64)).astype(np.float64)


def gelu_reference(x, approximate="none"):
    """GELU in float64; 'tanh' is the tanh approximation, else the erf form."""
    x = np.asarray(x, dtype=np.float64)
    if approximate == "tanh":
        return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))


_UNARY = {
    "neg": lambda x, a: np.negative(x),
    "exp": lambda x, a: np.exp(x),
    "tanh": lambda x, a: np.tanh(x),
    "sigmoid": lambda x, a: 1.0 / (1.0 + np.exp(-x)),
    "relu": lambda x, a: np.maximum(x, 0),
    "gelu": lambda x, a: gelu_reference(x, a.get("approximate", "none")),
    "rsqrt": lambda x, a: 1.0 / np.sqrt(x),
    "sqrt": lambda x, a: np.sqrt(x),
    "erf": lambda x, a: _erf(x),
    "copy": lambda x, a: np.array(x, copy=True),
}
_BINARY = {
    "add": np.add,
    "sub": np.subtract,
    "mul": np.multiply,
    "div": np.divide,
    "maximum": np.maximum,
    "minimum": np.minimum,
}

UNARY_OPS = tuple(_UNARY)
BINARY_OPS = tuple(_BINARY)


def _ew_infer(shapes, attrs):
    return broadcast_shapes(*shapes)


for _n, _f in _UNARY.items():
    _def(_n, "elementwise", _ew_infer, (lambda f: lambda xs, a: f(xs[0], a))(_f), 1)
for _n, _f in _BINARY.items():
    _def(_n, "elementwise", _ew_infer, (lambda f: lambda xs, a: f(xs[0], xs[1]))(_f), 2)


# reductions (keepdim) ------------------------------------------------------------

def _red_infer(shapes, attrs):
    (shape,) = shapes
    dims = {d % len(shape) for d in attrs["dims"]} if shape else set()
    return tuple(1 if i in dims else s for i, s in enumerate(shape))


_def("reduce_sum", "reduction", _red_infer,
     lambda xs, a: np.sum(xs[0], axis=tuple(a["dims"]), keepdims=True), 1)
_def("reduce_max", "reduction", _red_infer,
     lambda xs, a: np.max(xs[0], axis=tuple(a["dims"]), keepdims=True), 1)

REDUCTION_COMBINER = {"reduce_sum": "add", "reduce_max": "maximum"}
REDUCTION_INIT = {"reduce_sum": 0.0, "reduce_max": float("-inf")}


# matmul ----------------------------------------------------------------------------

def _mm_infer(shapes, attrs):
    a, b = shapes
    ok = len(a) == len(b) and len(a) in (2, 3) and a[-1] == b[-2] and a[:-2] == b[:-2]
    if not ok:
        raise ValueError(f"matmul: incompatible shapes {a} x {b}")
    return (*a[:-1], b[-1])


_def("matmul", "matmul", _mm_infer, lambda xs, a: np.matmul(xs[0], xs[1]), 2)


# views -------------------------------------------------------------------------------

def _transpose_infer(shapes, attrs):
    return tuple(shapes[0][p] for p in attrs["perm"])


def _reshape_infer(shapes, attrs):
    new = tuple(attrs["shape"])
    if prod(new) != prod(shapes[0]):
        raise ValueError(f"reshape: {shapes[0]} -> {new} changes element count")
    return new


def _slice_infer(shapes, attrs):
    out = list(shapes[0])
    d = attrs["dim"] % len(out)
    step = attrs.get("step", 1)
    start, end = attrs["start"], min(attrs["end"], out[d])
    out[d] = max(0, -(-(end - start) // step))
    return tuple(out)


def _slice_ref(xs, a):
    sl = [slice(None)] * xs[0].ndim
    sl[a["dim"]] = slice(a["start"], a["end"], a.get("step", 1))
    return xs[0][tuple(sl)]


def _expand_infer(shapes, attrs):
    return broadcast_shapes(shapes[0], tuple(attrs["shape"]))


_def("transpose", "view", _transpose_infer, lambda xs, a: np.transpose(xs[0], a["perm"]), 1)
_def("reshape", "view", _reshape_infer, lambda xs, a: np.reshape(xs[0], a["shape"]), 1)
_def("slice", "view", _slice_infer, _slice_ref, 1)
_def("expand", "view", _expand_infer, lambda xs, a: np.broadcast_to(xs[0], a["shape"]), 1)

_def("const", "const", lambda shapes, attrs: None, lambda xs, a: None, 0)


# helpers -------------------------------------------------------------------------------

def kind(op: str) -> str:
    return OPS[op].kind


def infer_type(op: str, input_types, attrs) -> TensorType:
    if op not in OPS:
        raise ValueError(f"unknown op '{op}'")
    d = OPS[op]
    if d.arity is not None and len(input_types) != d.arity:
        raise ValueError(f"{op} expects {d.arity} operands, got {len(input_types)}")
    shape = d.infer([t.shape for t in input_types], attrs)
    if shape is None:
        raise ValueError(f"{op}: result type must be given explicitly")
    return TensorType(tuple(int(s) for s in shape))


def evaluate(op: str, inputs, attrs) -> np.ndarray:
    """Evaluate one op on NumPy arrays; the result is a C-ordered f32 array."""
    out = OPS[op].ref([np.asarray(x) for x in inputs], attrs)
    return np.array(out, dtype=np.float32, order="C")


def interpret(graph: Graph, *inputs) -> list:
    """Run a whole graph with the NumPy semantics (for pass-level tests)."""
    user = [i for i, at in enumerate(graph.arg_attrs) if "param" not in at]
    if len(inputs) != len(user):
        raise ValueError(f"expected {len(user)} inputs, got {len(inputs)}")
    env = {}
    feed = iter(inputs)
    for arg, at in zip(graph.args, graph.arg_attrs):
        env[arg] = graph.constants[at["param"]] if "param" in at else np.asarray(next(feed), np.float32)
    for n in graph.nodes:
        if n.op == "const":
            env[n.out] = graph.const_data(n.out)
        else:
            env[n.out] = evaluate(n.op, [env[v] for v in n.inputs], n.attrs)
    return [env[v] for v in graph.results]
