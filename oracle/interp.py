"""Float64 NumPy interpreter of Kiln IR graphs.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Restates the reference's
op table, kiln/ir/ops.py:48-188, evaluated in float64 instead of rounding each
op to float32: elementwise ops with NumPy broadcasting (ops.py:55-74), keepdim
reductions (93-97), matmul on rank-2/3 operands (102-109), views as NumPy
views (114-146), gelu's tanh / erf forms (41-45).
"""

from __future__ import annotations

import math

import numpy as np

_erf = np.frompyfunc(math.erf, 1, 1)


def erf(x):
    return _erf(np.asarray(x, dtype=np.float64)).astype(np.float64)


def gelu(x, approximate="none"):
    if approximate == "tanh":
        return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def _eval(op, xs, at):
    x = xs[0] if xs else None
    with np.errstate(all="ignore"):
        if op == "add":
            return xs[0] + xs[1]
        if op == "sub":
            return xs[0] - xs[1]
        if op == "mul":
            return xs[0] * xs[1]
        if op == "div":
            return xs[0] / xs[1]
        if op == "maximum":
            return np.maximum(xs[0], xs[1])
        if op == "minimum":
            return np.minimum(xs[0], xs[1])
        if op == "neg":
            return -x
        if op == "exp":
            return np.exp(x)
        if op == "tanh":
            return np.tanh(x)
        if op == "sigmoid":
            return 1.0 / (1.0 + np.exp(-x))
        if op == "relu":
            return np.maximum(x, 0.0)
        if op == "gelu":
            return gelu(x, at.get("approximate", "none"))
        if op == "rsqrt":
            return 1.0 / np.sqrt(x)
        if op == "sqrt":
            return np.sqrt(x)
        if op == "erf":
            return erf(x)
        if op == "copy":
            return np.array(x, copy=True)
        if op == "reduce_sum":
            return np.sum(x, axis=tuple(at["dims"]), keepdims=True)
        if op == "reduce_max":
            return np.max(x, axis=tuple(at["dims"]), keepdims=True)
        if op == "matmul":
            return np.matmul(xs[0], xs[1])
        if op == "transpose":
            return np.transpose(x, at["perm"])
        if op == "reshape":
            return np.reshape(x, at["shape"])
        if op == "slice":
            sl = [slice(None)] * x.ndim
            sl[at["dim"]] = slice(at["start"], at["end"], at.get("step", 1))
            return x[tuple(sl)]
        if op == "expand":
            return np.broadcast_to(x, at["shape"])
    raise ValueError(f"oracle: unknown op {op}")


def run(graph, *inputs):
    """Evaluate `graph` on the user inputs (params come from graph.constants)."""
    env = {}
    feed = iter(inputs)
    for arg, at in zip(graph.args, graph.arg_attrs):
        data = graph.constants[at["param"]] if "param" in at else next(feed)
        env[arg] = np.asarray(data, dtype=np.float64)
    for n in graph.nodes:
        if n.op == "const":
            if "value" in n.attrs:
                env[n.out] = np.float64(n.attrs["value"])
            else:
                env[n.out] = np.asarray(graph.constants[n.attrs["name"]], dtype=np.float64)
        else:
            env[n.out] = _eval(n.op, [env[v] for v in n.inputs], n.attrs)
    return [np.asarray(env[v], dtype=np.float64) for v in graph.results]
