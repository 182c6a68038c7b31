"""The op set of the IR: for every op its kind, operand count, result shape
rule and NumPy meaning.

The names, attributes, kinds and result shapes are Kiln's (the reference's
kiln/ir/ops.py:48-188); the fusion pass, buffer assignment and the HIP
lowering dispatch on the kind. The NumPy meaning serves the constant folder
at compile time and ``interpret`` (a whole-graph evaluator for pass tests);
nothing on the GPU path calls it.

Kinds: ``elementwise`` (shapes broadcast NumPy-style), ``reduction``
(``dims``, always keepdim), ``matmul`` ([B,] M x K @ [B,] K x N), ``view``
(transpose / reshape / slice / expand: no data movement once buffers are
assigned) and ``const``.
"""

from __future__ import annotations

import math

import numpy as np

from kiln.ir.core import Graph, TensorType


class OpSpec:
    """kind, arity (None = any), shape(in_shapes, attrs) -> out shape or None,
    compute(arrays, attrs) -> array."""

    __slots__ = ("name", "kind", "arity", "shape", "compute")

    def __init__(self, name, kind, arity, shape, compute):
        self.name, self.kind, self.arity, self.shape, self.compute = name, kind, arity, shape, compute

    # kept for callers that read the fields by their older names
    infer = property(lambda self: self.shape)
    ref = property(lambda self: self.compute)


OPS: dict = {}


def _add(name, kind, arity, shape, compute):
    OPS[name] = OpSpec(name, kind, arity, shape, compute)


def broadcast_shapes(*shapes) -> tuple:
    return tuple(np.broadcast_shapes(*shapes))


# -- elementwise --------------------------------------------------------------------

_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
_erf_f64 = np.vectorize(math.erf, otypes=[np.float64])


def gelu_reference(x, approximate="none"):
    """GELU evaluated in float64: x * Phi(x), or with approximate="tanh"
    0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    x = np.asarray(x, dtype=np.float64)
    if approximate == "tanh":
        inner = _SQRT_2_OVER_PI * (x + 0.044715 * x * x * x)
        return 0.5 * x * (1.0 + np.tanh(inner))
    return 0.5 * x * (1.0 + _erf_f64(x * (1.0 / math.sqrt(2.0))))


def _unary(x, attrs, op):
    if op == "neg":
        return -x
    if op == "exp":
        return np.exp(x)
    if op == "tanh":
        return np.tanh(x)
    if op == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if op == "relu":
        return np.maximum(x, 0)
    if op == "gelu":
        return gelu_reference(x, attrs.get("approximate", "none"))
    if op == "rsqrt":
        return 1.0 / np.sqrt(x)
    if op == "sqrt":
        return np.sqrt(x)
    if op == "erf":
        return _erf_f64(x)
    if op == "copy":
        return np.array(x, copy=True)
    raise KeyError(op)


_BINARY_UFUNC = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide,
                 "maximum": np.maximum, "minimum": np.minimum}
UNARY_OPS = ("neg", "exp", "tanh", "sigmoid", "relu", "gelu", "rsqrt", "sqrt", "erf", "copy")
BINARY_OPS = tuple(_BINARY_UFUNC)


def _broadcast_rule(shapes, attrs):
    return broadcast_shapes(*shapes)


for _op in UNARY_OPS:
    _add(_op, "elementwise", 1, _broadcast_rule, lambda xs, attrs, _op=_op: _unary(xs[0], attrs, _op))
for _op, _ufunc in _BINARY_UFUNC.items():
    _add(_op, "elementwise", 2, _broadcast_rule, lambda xs, attrs, _u=_ufunc: _u(xs[0], xs[1]))


# -- reductions (keepdim) ---------------------------------------------------------------

def _reduced_shape(shapes, attrs):
    (shape,) = shapes
    rank = len(shape)
    gone = {d % rank for d in attrs["dims"]} if rank else set()
    return tuple(1 if d in gone else extent for d, extent in enumerate(shape))


_add("reduce_sum", "reduction", 1, _reduced_shape,
     lambda xs, attrs: xs[0].sum(axis=tuple(attrs["dims"]), keepdims=True))
_add("reduce_max", "reduction", 1, _reduced_shape,
     lambda xs, attrs: xs[0].max(axis=tuple(attrs["dims"]), keepdims=True))

# the elementwise op that combines two partial results, and its identity
REDUCTION_COMBINER = {"reduce_sum": "add", "reduce_max": "maximum"}
REDUCTION_INIT = {"reduce_sum": 0.0, "reduce_max": float("-inf")}


# -- matmul ---------------------------------------------------------------------------------

def _matmul_shape(shapes, attrs):
    a, b = shapes
    batch_ok = len(a) == len(b) and a[:-2] == b[:-2]
    if not (batch_ok and len(a) in (2, 3) and a[-1] == b[-2]):
        raise ValueError(f"matmul: incompatible shapes {a} x {b}")
    return tuple(a[:-1]) + (b[-1],)


_add("matmul", "matmul", 2, _matmul_shape, lambda xs, attrs: xs[0] @ xs[1])


# -- views ------------------------------------------------------------------------------------

def _transpose_shape(shapes, attrs):
    src = shapes[0]
    return tuple(src[axis] for axis in attrs["perm"])


def _reshape_shape(shapes, attrs):
    target = tuple(attrs["shape"])
    if math.prod(target) != math.prod(shapes[0]):
        raise ValueError(f"reshape: {shapes[0]} -> {target} changes element count")
    return target


def _slice_shape(shapes, attrs):
    dims = list(shapes[0])
    d = attrs["dim"] % len(dims)
    lo, hi, step = attrs["start"], min(attrs["end"], dims[d]), attrs.get("step", 1)
    dims[d] = len(range(lo, hi, step)) if hi > lo else 0
    return tuple(dims)


def _slice_compute(xs, attrs):
    x = xs[0]
    index = tuple(slice(attrs["start"], attrs["end"], attrs.get("step", 1)) if d == attrs["dim"] % x.ndim
                  else slice(None) for d in range(x.ndim))
    return x[index]


_add("transpose", "view", 1, _transpose_shape, lambda xs, attrs: np.transpose(xs[0], attrs["perm"]))
_add("reshape", "view", 1, _reshape_shape, lambda xs, attrs: np.reshape(xs[0], tuple(attrs["shape"])))
_add("slice", "view", 1, _slice_shape, _slice_compute)
_add("expand", "view", 1, lambda shapes, attrs: broadcast_shapes(shapes[0], tuple(attrs["shape"])),
     lambda xs, attrs: np.broadcast_to(xs[0], tuple(attrs["shape"])))

# const: its type is always given explicitly, its data comes from the graph
_add("const", "const", 0, lambda shapes, attrs: None, lambda xs, attrs: None)


# -- queries ------------------------------------------------------------------------------------

def kind(op: str) -> str:
    return OPS[op].kind


def infer_type(op: str, input_types, attrs) -> TensorType:
    spec = OPS.get(op)
    if spec is None:
        raise ValueError(f"unknown op '{op}'")
    if spec.arity is not None and len(input_types) != spec.arity:
        raise ValueError(f"{op} expects {spec.arity} operands, got {len(input_types)}")
    shape = spec.shape([t.shape for t in input_types], attrs)
    if shape is None:
        raise ValueError(f"{op}: result type must be given explicitly")
    return TensorType(tuple(map(int, shape)))


def evaluate(op: str, inputs, attrs) -> np.ndarray:
    """One op on NumPy arrays; always returns a C-contiguous float32 array
    (0-d for a scalar result)."""
    result = OPS[op].compute([np.asarray(x) for x in inputs], attrs)
    return np.array(result, dtype=np.float32, order="C")


def interpret(graph: Graph, *inputs) -> list:
    """Evaluate the whole graph with the NumPy meaning of each op. ``inputs``
    feed the non-``param`` arguments in order; ``param`` arguments read their
    data from ``graph.constants``."""
    runtime = [i for i, attrs in enumerate(graph.arg_attrs) if "param" not in attrs]
    if len(inputs) != len(runtime):
        raise ValueError(f"expected {len(runtime)} inputs, got {len(inputs)}")
    values = {}
    for arg, attrs in zip(graph.args, graph.arg_attrs):
        if "param" in attrs:
            values[arg] = graph.constants[attrs["param"]]
    for i, x in zip(runtime, inputs):
        values[graph.args[i]] = np.asarray(x, np.float32)
    for node in graph.nodes:
        if node.op == "const":
            values[node.out] = graph.const_data(node.out)
        else:
            values[node.out] = evaluate(node.op, [values[v] for v in node.inputs], node.attrs)
    return [values[v] for v in graph.results]
