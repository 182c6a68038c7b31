"""Import ATen-level torch.fx graphs (from ``torch.export``) into the Kiln IR.

The decompositions are part of the backend contract: they decide which op
sequences the fusion pass hands to each HIP kernel family, and the HIP
lowering pattern-matches them (LayerNorm, softmax, bias + GELU). They follow
the reference frontend (kiln/frontend/fx_import.py:92-288):

  linear/addmm   -> transpose(W) + matmul + add(bias)
  softmax        -> reduce_max, sub, exp, reduce_sum, div
  layer_norm     -> reduce_sum * (1/n), sub, mul(xc, xc), reduce_sum * (1/n),
                    add eps, rsqrt, mul, [mul gamma], [add beta]
  gelu           -> gelu {approximate}
  pow(x, 2)      -> mul(x, x)
  mean           -> reduce_sum * (1/count)

Anything else raises ``Unsupported`` (a NotImplementedError).
"""

from __future__ import annotations

import operator
from numbers import Number

import numpy as np
import torch
import torch.fx

from kiln.ir.core import Graph, TensorType, Value, verify

aten = torch.ops.aten


class Unsupported(NotImplementedError):
    """The graph uses something Kiln cannot compile."""


def _static_shape(node) -> tuple:
    val = node.meta.get("val")
    if not isinstance(val, torch.Tensor):
        raise Unsupported(f"{node.name}: no tensor metadata")
    if val.dtype != torch.float32:
        raise Unsupported(f"{node.name}: only float32 is supported (got {val.dtype})")
    if not all(isinstance(d, int) for d in val.shape):
        raise Unsupported(f"{node.name}: dynamic shapes are not supported")
    return tuple(val.shape)


_BINARY = {
    aten.add.Tensor: "add", aten.add.Scalar: "add",
    aten.sub.Tensor: "sub", aten.sub.Scalar: "sub",
    aten.mul.Tensor: "mul", aten.mul.Scalar: "mul",
    aten.div.Tensor: "div", aten.div.Scalar: "div",
    aten.maximum.default: "maximum", aten.minimum.default: "minimum",
}
_UNARY = {
    aten.neg.default: "neg", aten.exp.default: "exp", aten.tanh.default: "tanh",
    aten.sigmoid.default: "sigmoid", aten.relu.default: "relu", aten.rsqrt.default: "rsqrt",
    aten.sqrt.default: "sqrt", aten.erf.default: "erf",
}
_IDENTITY = (aten.clone.default, aten.alias.default, aten.detach.default,
             aten.lift_fresh_copy.default, aten.contiguous.default)
_RESHAPES = (aten.view.default, aten.reshape.default, aten._unsafe_view.default,
             aten.unsqueeze.default, aten.squeeze.dim, aten.squeeze.dims, aten.squeeze.default,
             aten.flatten.using_ints)


class _Importer:
    def __init__(self, name):
        self.g = Graph(name)
        self.env = {}
        self.scalar_cache = {}

    # operands -----------------------------------------------------------------

    def val(self, arg) -> Value:
        if isinstance(arg, torch.fx.Node):
            v = self.env[arg]
            if not isinstance(v, Value):
                raise Unsupported(f"{arg.name}: expected a single tensor")
            return v
        if isinstance(arg, bool) or not isinstance(arg, Number):
            raise Unsupported(f"unsupported operand {arg!r}")
        key = float(arg)
        if key not in self.scalar_cache:
            self.scalar_cache[key] = self.g.scalar(key)
        return self.scalar_cache[key]

    def emit(self, op, *inputs, **attrs) -> Value:
        return self.g.add_node(op, list(inputs), attrs)

    def reduce(self, op, x: Value, dims) -> Value:
        return self.emit(op, x, dims=sorted(d % x.type.rank for d in dims))

    def drop_dims(self, x: Value, dims) -> Value:
        gone = set(dims)
        return self.emit("reshape", x, shape=[s for i, s in enumerate(x.shape) if i not in gone])

    def mean(self, x: Value, dims, keepdim=True) -> Value:
        dims = sorted(d % x.type.rank for d in dims)
        count = int(np.prod([x.shape[d] for d in dims]))
        m = self.emit("mul", self.reduce("reduce_sum", x, dims), self.val(1.0 / count))
        return m if keepdim else self.drop_dims(m, dims)

    def matmul(self, a, b, bias=None) -> Value:
        out = self.emit("matmul", a, b)
        return self.emit("add", out, bias) if bias is not None else out

    @staticmethod
    def _keepdim(args, kw):
        return args[2] if len(args) > 2 else kw.get("keepdim", False)

    # conversion ---------------------------------------------------------------

    def convert(self, node: torch.fx.Node):
        t, args, kw = node.target, node.args, node.kwargs
        if t is operator.getitem:
            return self.env[args[0]][args[1]]
        if t in _IDENTITY:
            return self.val(args[0])
        if t in _BINARY:
            a, b = self.val(args[0]), self.val(args[1])
            alpha = kw.get("alpha", 1)
            if alpha != 1:
                b = self.emit("mul", b, self.val(alpha))
            return self.emit(_BINARY[t], a, b)
        if t is aten.rsub.Scalar:
            return self.emit("sub", self.val(args[1]), self.val(args[0]))
        if t in _UNARY:
            return self.emit(_UNARY[t], self.val(args[0]))
        if t is aten.gelu.default:
            return self.emit("gelu", self.val(args[0]), approximate=kw.get("approximate", "none"))
        if t is aten.pow.Tensor_Scalar and args[1] == 2:
            x = self.val(args[0])
            return self.emit("mul", x, x)
        if t in (aten.mm.default, aten.bmm.default):
            return self.emit("matmul", self.val(args[0]), self.val(args[1]))
        if t is aten.addmm.default:
            if kw.get("beta", 1) != 1 or kw.get("alpha", 1) != 1:
                raise Unsupported("addmm with alpha/beta != 1")
            return self.matmul(self.val(args[1]), self.val(args[2]), self.val(args[0]))
        if t is aten.linear.default:
            return self.linear(args)
        return self.convert_view_or_composite(node, t, args, kw)

    def linear(self, args):
        x, w = self.val(args[0]), self.val(args[1])
        bias = self.val(args[2]) if len(args) > 2 and args[2] is not None else None
        wt = self.emit("transpose", w, perm=[1, 0])
        if x.type.rank == 2:
            return self.matmul(x, wt, bias)
        lead = list(x.shape[:-1])
        flat = self.emit("reshape", x, shape=[int(np.prod(lead)), x.shape[-1]])
        return self.emit("reshape", self.matmul(flat, wt, bias), shape=[*lead, w.shape[0]])

    def convert_view_or_composite(self, node, t, args, kw):
        if t is aten.t.default:
            x = self.val(args[0])
            return x if x.type.rank < 2 else self.emit("transpose", x, perm=[1, 0])
        if t is aten.permute.default:
            return self.emit("transpose", self.val(args[0]), perm=[d % len(args[1]) for d in args[1]])
        if t is aten.transpose.int:
            x = self.val(args[0])
            perm = list(range(x.type.rank))
            i, j = args[1] % x.type.rank, args[2] % x.type.rank
            perm[i], perm[j] = perm[j], perm[i]
            return self.emit("transpose", x, perm=perm)
        if t in _RESHAPES:
            return self.emit("reshape", self.val(args[0]), shape=list(_static_shape(node)))
        if t is aten.expand.default:
            return self.emit("expand", self.val(args[0]), shape=list(_static_shape(node)))
        if t is aten.slice.Tensor:
            x = self.val(args[0])
            dim = (args[1] if len(args) > 1 else 0) % x.type.rank
            size = x.shape[dim]
            start = args[2] if len(args) > 2 and args[2] is not None else 0
            end = args[3] if len(args) > 3 and args[3] is not None else size
            step = args[4] if len(args) > 4 else 1
            start = start + size if start < 0 else start
            end = end + size if end < 0 else end
            return self.emit("slice", x, dim=dim, start=max(0, start), end=min(end, size), step=step)
        if t is aten.select.int:
            # x[..., i, ...]: a one-element slice, then the dim dropped (both views)
            x = self.val(args[0])
            dim = args[1] % x.type.rank
            i = args[2] + x.shape[dim] if args[2] < 0 else args[2]
            one = self.emit("slice", x, dim=dim, start=i, end=i + 1, step=1)
            return self.drop_dims(one, [dim])
        if t in (aten.split_with_sizes.default, aten.split.Tensor):
            x = self.val(args[0])
            dim = (args[2] if len(args) > 2 else kw.get("dim", 0)) % x.type.rank
            sizes = args[1]
            if isinstance(sizes, int):
                n = x.shape[dim]
                sizes = [min(sizes, n - i) for i in range(0, n, sizes)]
            pieces, start = [], 0
            for s in sizes:
                pieces.append(self.emit("slice", x, dim=dim, start=start, end=start + s, step=1))
                start += s
            return pieces
        if t in (aten.sum.dim_IntList, aten.amax.default):
            x = self.val(args[0])
            op = "reduce_sum" if t is aten.sum.dim_IntList else "reduce_max"
            out = self.reduce(op, x, args[1])
            if self._keepdim(args, kw):
                return out
            return self.drop_dims(out, [d % x.type.rank for d in args[1]])
        if t is aten.mean.dim:
            return self.mean(self.val(args[0]), args[1], self._keepdim(args, kw))
        if t is aten._softmax.default:
            x = self.val(args[0])
            dim = args[1] % node.args[0].meta["val"].dim()
            shifted = self.emit("sub", x, self.reduce("reduce_max", x, [dim]))
            e = self.emit("exp", shifted)
            return self.emit("div", e, self.reduce("reduce_sum", e, [dim]))
        if t is aten.native_layer_norm.default:
            return self.layer_norm(args)
        raise Unsupported(f"Kiln does not support {t} yet")

    def layer_norm(self, args):
        x, normalized, weight, bias, eps = self.val(args[0]), args[1], args[2], args[3], args[4]
        dims = list(range(x.type.rank - len(normalized), x.type.rank))
        mean = self.mean(x, dims)
        xc = self.emit("sub", x, mean)
        var = self.mean(self.emit("mul", xc, xc), dims)
        rstd = self.emit("rsqrt", self.emit("add", var, self.val(eps)))
        y = self.emit("mul", xc, rstd)
        if weight is not None:
            y = self.emit("mul", y, self.val(weight))
        if bias is not None:
            y = self.emit("add", y, self.val(bias))
        return (y, mean, rstd)

    # driver ---------------------------------------------------------------------

    def run(self, gm: torch.fx.GraphModule, params=None) -> Graph:
        params = params or {}
        for node in gm.graph.nodes:
            if node.op == "placeholder":
                shape = TensorType(_static_shape(node))
                if node.name in params:
                    pname, data = params[node.name]
                    self.g.constants[pname] = data
                    self.env[node] = self.g.add_arg(shape, pname, param=pname)
                else:
                    self.env[node] = self.g.add_arg(shape, node.name)
            elif node.op == "call_function":
                out = self.convert(node)
                self.env[node] = out
                if isinstance(out, Value) and isinstance(node.meta.get("val"), torch.Tensor):
                    want = _static_shape(node)
                    if tuple(out.shape) != want:
                        raise AssertionError(f"{node.name}: Kiln shape {out.shape} != {want}")
            elif node.op == "output":
                outs = node.args[0]
                outs = list(outs) if isinstance(outs, (list, tuple)) else [outs]
                if not all(isinstance(o, torch.fx.Node) for o in outs):
                    raise Unsupported("graph returns non-tensor outputs")
                self.g.results = [self.val(o) for o in outs]
            else:
                raise Unsupported(f"unsupported FX node kind '{node.op}'")
        verify(self.g)
        return self.g


def import_fx(gm: torch.fx.GraphModule, name="forward") -> Graph:
    """An aot_autograd forward graph: every placeholder is a runtime input."""
    return _Importer(name).run(gm)


def import_exported(ep, name="forward") -> Graph:
    """A decomposed ``torch.export.ExportedProgram``; parameters, buffers and
    constant tensors become ``param`` arguments the freeze pass can fold."""
    from torch.export.graph_signature import InputKind, OutputKind

    params = {}
    for spec in ep.graph_signature.input_specs:
        if spec.kind in (InputKind.PARAMETER, InputKind.BUFFER, InputKind.CONSTANT_TENSOR):
            t = ep.state_dict.get(spec.target)
            if t is None:
                t = ep.constants[spec.target]
            params[spec.arg.name] = (spec.target, t.detach().to(torch.float32).cpu().numpy().copy())
        elif spec.kind != InputKind.USER_INPUT:
            raise Unsupported(f"unsupported graph input kind {spec.kind}")
    for spec in ep.graph_signature.output_specs:
        if spec.kind != OutputKind.USER_OUTPUT:
            raise Unsupported(f"unsupported graph output kind {spec.kind} (mutation?)")
    return _Importer(name).run(ep.graph_module, params)
