"""From ATen-level torch.fx graphs (``torch.export`` after
``run_decompositions()``, or an aot_autograd forward graph) to the IR.

Each supported ATen overload has a translator registered in ``_TRANSLATORS``.
Composite ops are expanded into IR ops by the ``expand_*`` recipes below. The
recipes are Kiln's decompositions (the reference's
kiln/frontend/fx_import.py:128-153, 212-230), node for node and in the same
order, because they fix which op sequences fusion hands to a kernel family
and the HIP lowering recognises them (LayerNorm, softmax, bias + GELU):

  linear / addmm  transpose(W) [reshape], matmul, add(bias) [reshape back]
  softmax         reduce_max, sub, exp, reduce_sum, div
  layer_norm      reduce_sum, *1/n, sub, mul(xc, xc), reduce_sum, *1/n,
                  add(eps), rsqrt, mul, [mul(gamma)], [add(beta)]
  mean            reduce_sum, mul(1/count)
  pow(x, 2)       mul(x, x)

Python numbers become scalar constants, one per distinct value, created where
first used. Anything without a translator raises ``Unsupported`` (a
NotImplementedError).
"""

from __future__ import annotations

import math
import operator
from numbers import Number

import torch
import torch.fx

from kiln.ir.core import Graph, TensorType, Value, verify

aten = torch.ops.aten


class Unsupported(NotImplementedError):
    """The graph uses something Kiln cannot compile."""


def static_shape(node: torch.fx.Node) -> tuple:
    meta = node.meta.get("val")
    if not isinstance(meta, torch.Tensor):
        raise Unsupported(f"{node.name}: no tensor metadata")
    if meta.dtype != torch.float32:
        raise Unsupported(f"{node.name}: only float32 is supported (got {meta.dtype})")
    dims = tuple(meta.shape)
    if any(not isinstance(d, int) for d in dims):
        raise Unsupported(f"{node.name}: dynamic shapes are not supported")
    return dims


class _Builder:
    """Appends IR nodes to a graph; turns Python numbers into scalar consts."""

    def __init__(self, graph: Graph):
        self.graph = graph
        self._scalars = {}

    def number(self, x) -> Value:
        if isinstance(x, bool) or not isinstance(x, Number):
            raise Unsupported(f"unsupported operand {x!r}")
        key = float(x)
        if key not in self._scalars:
            self._scalars[key] = self.graph.scalar(key)
        return self._scalars[key]

    def __call__(self, op: str, *inputs: Value, **attrs) -> Value:
        return self.graph.add_node(op, list(inputs), attrs)

    def reduce(self, op: str, x: Value, dims) -> Value:
        return self(op, x, dims=sorted(d % x.type.rank for d in dims))

    def squeeze(self, x: Value, dims) -> Value:
        return self("reshape", x, shape=[e for d, e in enumerate(x.shape) if d not in set(dims)])


# -- decomposition recipes --------------------------------------------------------------------

def expand_mean(b: _Builder, x: Value, dims, keepdim=True) -> Value:
    dims = sorted(d % x.type.rank for d in dims)
    total = b.reduce("reduce_sum", x, dims)
    mean = b("mul", total, b.number(1.0 / math.prod(x.shape[d] for d in dims)))
    return mean if keepdim else b.squeeze(mean, dims)


def expand_linear(b: _Builder, x: Value, w: Value, bias: Value | None) -> Value:
    wt = b("transpose", w, perm=[1, 0])
    if x.type.rank == 2:
        return expand_matmul_bias(b, x, wt, bias)
    rows = math.prod(x.shape[:-1])
    flat = b("reshape", x, shape=[rows, x.shape[-1]])
    out = expand_matmul_bias(b, flat, wt, bias)
    return b("reshape", out, shape=[*x.shape[:-1], w.shape[0]])


def expand_matmul_bias(b: _Builder, a: Value, w: Value, bias: Value | None) -> Value:
    product = b("matmul", a, w)
    return product if bias is None else b("add", product, bias)


def expand_softmax(b: _Builder, x: Value, dim: int) -> Value:
    shifted = b("sub", x, b.reduce("reduce_max", x, [dim]))
    e = b("exp", shifted)
    return b("div", e, b.reduce("reduce_sum", e, [dim]))


def expand_layer_norm(b: _Builder, x: Value, n_norm: int, gamma, beta, eps):
    dims = list(range(x.type.rank - n_norm, x.type.rank))
    mean = expand_mean(b, x, dims)
    centred = b("sub", x, mean)
    var = expand_mean(b, b("mul", centred, centred), dims)
    rstd = b("rsqrt", b("add", var, b.number(eps)))
    y = b("mul", centred, rstd)
    if gamma is not None:
        y = b("mul", y, gamma)
    if beta is not None:
        y = b("add", y, beta)
    return y, mean, rstd


# -- translators ----------------------------------------------------------------------------------

_TRANSLATORS = {}


def translates(*targets):
    def register(fn):
        for t in targets:
            _TRANSLATORS[t] = fn
        return fn

    return register


def _arg(args, i, default=None):
    return args[i] if len(args) > i and args[i] is not None else default


_ELEMENTWISE = {
    aten.add.Tensor: "add", aten.add.Scalar: "add", aten.sub.Tensor: "sub", aten.sub.Scalar: "sub",
    aten.mul.Tensor: "mul", aten.mul.Scalar: "mul", aten.div.Tensor: "div", aten.div.Scalar: "div",
    aten.maximum.default: "maximum", aten.minimum.default: "minimum",
    aten.neg.default: "neg", aten.exp.default: "exp", aten.tanh.default: "tanh",
    aten.sigmoid.default: "sigmoid", aten.relu.default: "relu", aten.rsqrt.default: "rsqrt",
    aten.sqrt.default: "sqrt", aten.erf.default: "erf",
}


@translates(*_ELEMENTWISE)
def _elementwise(t, node, args, kwargs):
    operands = [t.value(a) for a in args]
    scale = kwargs.get("alpha", 1)
    if scale != 1:
        operands[1] = t.b("mul", operands[1], t.value(scale))
    return t.b(_ELEMENTWISE[node.target], *operands)


@translates(aten.clone.default, aten.alias.default, aten.detach.default, aten.lift_fresh_copy.default,
            aten.contiguous.default)
def _passthrough(t, node, args, kwargs):
    return t.value(args[0])


@translates(operator.getitem)
def _getitem(t, node, args, kwargs):
    return t.env[args[0]][args[1]]


@translates(aten.rsub.Scalar)
def _rsub(t, node, args, kwargs):
    x, s = t.value(args[0]), t.value(args[1])
    return t.b("sub", s, x)


@translates(aten.gelu.default)
def _gelu(t, node, args, kwargs):
    return t.b("gelu", t.value(args[0]), approximate=kwargs.get("approximate", "none"))


@translates(aten.pow.Tensor_Scalar)
def _pow(t, node, args, kwargs):
    if args[1] != 2:
        raise Unsupported(f"pow with exponent {args[1]!r} (only 2 is supported)")
    x = t.value(args[0])
    return t.b("mul", x, x)


@translates(aten.mm.default, aten.bmm.default)
def _matmul(t, node, args, kwargs):
    return t.b("matmul", t.value(args[0]), t.value(args[1]))


@translates(aten.addmm.default)
def _addmm(t, node, args, kwargs):
    if kwargs.get("beta", 1) != 1 or kwargs.get("alpha", 1) != 1:
        raise Unsupported("addmm with alpha/beta != 1")
    a, w, bias = t.value(args[1]), t.value(args[2]), t.value(args[0])
    return expand_matmul_bias(t.b, a, w, bias)


@translates(aten.linear.default)
def _linear(t, node, args, kwargs):
    x, w = t.value(args[0]), t.value(args[1])
    bias = _arg(args, 2)
    return expand_linear(t.b, x, w, None if bias is None else t.value(bias))


@translates(aten.t.default)
def _t(t, node, args, kwargs):
    x = t.value(args[0])
    return x if x.type.rank < 2 else t.b("transpose", x, perm=[1, 0])


@translates(aten.permute.default)
def _permute(t, node, args, kwargs):
    axes = args[1]
    return t.b("transpose", t.value(args[0]), perm=[a % len(axes) for a in axes])


@translates(aten.transpose.int)
def _swap_axes(t, node, args, kwargs):
    x = t.value(args[0])
    r = x.type.rank
    i, j = args[1] % r, args[2] % r
    perm = [j if d == i else i if d == j else d for d in range(r)]
    return t.b("transpose", x, perm=perm)


@translates(aten.view.default, aten.reshape.default, aten._unsafe_view.default, aten.unsqueeze.default,
            aten.squeeze.dim, aten.squeeze.dims, aten.squeeze.default, aten.flatten.using_ints)
def _reshape(t, node, args, kwargs):
    return t.b("reshape", t.value(args[0]), shape=list(static_shape(node)))


@translates(aten.expand.default)
def _expand(t, node, args, kwargs):
    return t.b("expand", t.value(args[0]), shape=list(static_shape(node)))


@translates(aten.slice.Tensor)
def _slice(t, node, args, kwargs):
    x = t.value(args[0])
    dim = _arg(args, 1, 0) % x.type.rank
    size = x.shape[dim]
    lo, hi, step = _arg(args, 2, 0), _arg(args, 3, size), _arg(args, 4, 1)
    lo, hi = (lo + size if lo < 0 else lo), (hi + size if hi < 0 else hi)
    return t.b("slice", x, dim=dim, start=max(0, lo), end=min(hi, size), step=step)


@translates(aten.select.int)
def _select(t, node, args, kwargs):
    x = t.value(args[0])
    dim = args[1] % x.type.rank
    at = args[2] % x.shape[dim] if args[2] < 0 else args[2]
    one = t.b("slice", x, dim=dim, start=at, end=at + 1, step=1)
    return t.b.squeeze(one, [dim])


@translates(aten.split_with_sizes.default, aten.split.Tensor)
def _split(t, node, args, kwargs):
    x = t.value(args[0])
    dim = _arg(args, 2, kwargs.get("dim", 0)) % x.type.rank
    size = x.shape[dim]
    sizes = args[1]
    if isinstance(sizes, int):
        sizes = [min(sizes, size - lo) for lo in range(0, size, sizes)]
    starts = [sum(sizes[:k]) for k in range(len(sizes))]
    return [t.b("slice", x, dim=dim, start=lo, end=lo + n, step=1) for lo, n in zip(starts, sizes)]


@translates(aten.sum.dim_IntList, aten.amax.default)
def _reduce(t, node, args, kwargs):
    x = t.value(args[0])
    op = "reduce_max" if node.target is aten.amax.default else "reduce_sum"
    out = t.b.reduce(op, x, args[1])
    keepdim = _arg(args, 2, kwargs.get("keepdim", False))
    return out if keepdim else t.b.squeeze(out, [d % x.type.rank for d in args[1]])


@translates(aten.mean.dim)
def _mean(t, node, args, kwargs):
    return expand_mean(t.b, t.value(args[0]), args[1], _arg(args, 2, kwargs.get("keepdim", False)))


@translates(aten._softmax.default)
def _softmax(t, node, args, kwargs):
    x = t.value(args[0])
    return expand_softmax(t.b, x, args[1] % x.type.rank)


@translates(aten.native_layer_norm.default)
def _layer_norm(t, node, args, kwargs):
    x = t.value(args[0])
    gamma = None if args[2] is None else t.value(args[2])
    beta = None if args[3] is None else t.value(args[3])
    return expand_layer_norm(t.b, x, len(args[1]), gamma, beta, args[4])


# -- the graph walk ---------------------------------------------------------------------------------

class _Translator:
    def __init__(self, name: str):
        self.graph = Graph(name)
        self.b = _Builder(self.graph)
        self.env = {}

    def value(self, x) -> Value:
        """The IR value of an FX operand (a node's single tensor) or number."""
        if not isinstance(x, torch.fx.Node):
            return self.b.number(x)
        v = self.env[x]
        if not isinstance(v, Value):
            raise Unsupported(f"{x.name}: expected a single tensor")
        return v

    def placeholder(self, node, params):
        t = TensorType(static_shape(node))
        if node.name in params:
            target, data = params[node.name]
            self.graph.constants[target] = data
            return self.graph.add_arg(t, target, param=target)
        return self.graph.add_arg(t, node.name)

    def call(self, node):
        translate = _TRANSLATORS.get(node.target)
        if translate is None:
            raise Unsupported(f"Kiln does not support {node.target} yet")
        out = translate(self, node, node.args, node.kwargs)
        if isinstance(out, Value) and isinstance(node.meta.get("val"), torch.Tensor):
            if tuple(out.shape) != static_shape(node):
                raise AssertionError(f"{node.name}: Kiln shape {out.shape} != {static_shape(node)}")
        return out

    def output(self, node):
        outs = node.args[0]
        outs = list(outs) if isinstance(outs, (list, tuple)) else [outs]
        if any(not isinstance(o, torch.fx.Node) for o in outs):
            raise Unsupported("graph returns non-tensor outputs")
        return [self.value(o) for o in outs]

    def run(self, gm: torch.fx.GraphModule, params=None) -> Graph:
        params = params or {}
        for node in gm.graph.nodes:
            if node.op == "placeholder":
                self.env[node] = self.placeholder(node, params)
            elif node.op == "call_function":
                self.env[node] = self.call(node)
            elif node.op == "output":
                self.graph.results = self.output(node)
            else:
                raise Unsupported(f"unsupported FX node kind '{node.op}'")
        verify(self.graph)
        return self.graph


def import_fx(gm: torch.fx.GraphModule, name="forward") -> Graph:
    """An aot_autograd forward graph: every placeholder is a runtime input."""
    return _Translator(name).run(gm)


def import_exported(ep, name="forward") -> Graph:
    """A decomposed ``torch.export.ExportedProgram``. Parameters, buffers and
    constant tensors become ``param`` arguments (named by their state-dict
    key), which the freeze pass turns into constants."""
    from torch.export.graph_signature import InputKind, OutputKind

    weights = (InputKind.PARAMETER, InputKind.BUFFER, InputKind.CONSTANT_TENSOR)
    params = {}
    for spec in ep.graph_signature.input_specs:
        if spec.kind in weights:
            tensor = ep.state_dict[spec.target] if spec.target in ep.state_dict else ep.constants[spec.target]
            params[spec.arg.name] = (spec.target, tensor.detach().to(torch.float32).cpu().numpy().copy())
        elif spec.kind != InputKind.USER_INPUT:
            raise Unsupported(f"unsupported graph input kind {spec.kind}")
    bad = [s.kind for s in ep.graph_signature.output_specs if s.kind != OutputKind.USER_OUTPUT]
    if bad:
        raise Unsupported(f"unsupported graph output kind {bad[0]} (mutation?)")
    return _Translator(name).run(ep.graph_module, params)
