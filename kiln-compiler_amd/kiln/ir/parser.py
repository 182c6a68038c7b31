"""Parser for the textual Kiln IR printed by kiln/ir/printer.py.

Accepts the reference's grammar (kiln/ir/parser.py:17-234). Constants or
``param`` arguments written without data get deterministic data derived from
their name, N(0, 1) * 0.1 drawn from ``numpy.random.default_rng(crc32(name))``
(the same rule as the reference's parser.py:225-227, so hand-written IR
compiles to the same numbers in both).
"""

from __future__ import annotations

import re
import zlib

import numpy as np

from kiln.ir.core import Graph, Kernel, Node, TensorType


class ParseError(ValueError):
    pass


_LEX = re.compile(r"""
    (?P<ws>\s+) | (?P<comment>//[^\n]*)
  | (?P<value>%[A-Za-z0-9_.]+) | (?P<symbol>@[A-Za-z0-9_.]+)
  | (?P<string>"(?:[^"\\]|\\.)*")
  | (?P<number>[-+]?(?:\d+\.\d*(?:[eE][-+]?\d+)?|\d+[eE][-+]?\d+|\d+|inf|nan)(?![A-Za-z_]))
  | (?P<arrow>->) | (?P<ident>[A-Za-z_][A-Za-z0-9_.]*) | (?P<punct>[{}()\[\],:=])
""", re.VERBOSE)


def _lex(text):
    toks, pos, line = [], 0, 1
    while pos < len(text):
        m = _LEX.match(text, pos)
        if m is None:
            raise ParseError(f"line {line}: unexpected character {text[pos]!r}")
        kind = m.lastgroup
        if kind not in ("ws", "comment"):
            toks.append((kind, m.group(), line))
        line += m.group().count("\n")
        pos = m.end()
    toks.append(("eof", None, line))
    return toks


def fake_data(name: str, shape) -> np.ndarray:
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    return rng.standard_normal(shape).astype(np.float32) * 0.1


class _Reader:
    def __init__(self, text):
        self.toks = _lex(text)
        self.pos = 0

    @property
    def tok(self):
        return self.toks[self.pos]

    def take(self):
        t = self.toks[self.pos]
        self.pos += 1
        return t

    def need(self, text=None, kind=None):
        k, v, line = self.take()
        if (text is not None and v != text) or (kind is not None and k != kind):
            raise ParseError(f"line {line}: expected {text if text is not None else kind!r}, got {v!r}")
        return v

    def maybe(self, text):
        if self.tok[1] == text:
            self.pos += 1
            return True
        return False

    def comma_list(self, close, item):
        items = []
        if self.maybe(close):
            return items
        while True:
            items.append(item())
            if self.maybe(close):
                return items
            self.need(",")

    # attributes / types ---------------------------------------------------------

    def value_attr(self):
        k, v, line = self.take()
        if k == "number":
            is_float = any(c in v for c in ".eEn") or v.lstrip("+-") == "inf"
            return float(v) if is_float else int(v)
        if k == "string":
            return bytes(v[1:-1], "utf-8").decode("unicode_escape")
        if k == "ident" and v in ("true", "false"):
            return v == "true"
        if v == "[":
            return self.comma_list("]", self.value_attr)
        if v == "{":
            self.pos -= 1
            return self.attr_dict()
        raise ParseError(f"line {line}: bad attribute value {v!r}")

    def attr_dict(self):
        if self.tok[1] != "{":
            return {}
        self.take()
        out = {}

        def entry():
            key = self.need(kind="ident")
            self.need("=")
            out[key] = self.value_attr()

        self.comma_list("}", entry)
        return out

    def tensor_type(self):
        dtype = self.need(kind="ident")
        self.need("[")
        dims = self.comma_list("]", lambda: int(self.need(kind="number")))
        return TensorType(tuple(dims), dtype)

    # graph --------------------------------------------------------------------------

    def graph(self) -> Graph:
        self.need("graph")
        g = Graph(self.need(kind="symbol")[1:])
        env = {}

        def arg():
            vname = self.need(kind="value")
            self.need(":")
            t = self.tensor_type()
            at = self.attr_dict()
            env[vname] = g.add_arg(t, at.get("param", vname[1:]), **at)

        self.need("(")
        self.comma_list(")", arg)
        self.need("->")
        self.need("(")
        self.comma_list(")", self.tensor_type)
        if self.maybe("attributes"):
            g.attrs = self.attr_dict()
        self.need("{")
        while True:
            k, v, line = self.tok
            if v == "kernel":
                self.take()
                kname = self.need(kind="symbol")[1:]
                kkind = self.need(kind="ident")
                g.kernels.append(Kernel(kname, kkind, [], self.attr_dict()))
            elif v == "return":
                self.take()
                res = []
                if self.tok[0] == "value":
                    res.append(self.lookup(env))
                    while self.maybe(","):
                        res.append(self.lookup(env))
                g.results = res
                self.need("}")
                break
            elif k == "value":
                self.node(g, env)
            else:
                raise ParseError(f"line {line}: unexpected {v!r}")

        by_name = {k.name: k for k in g.kernels}
        for n in g.nodes:
            kname = n.attrs.get("kernel")
            if kname is not None:
                if kname not in by_name:
                    raise ParseError(f"node refers to undeclared kernel @{kname}")
                by_name[kname].nodes.append(n)
        for a, at in zip(g.args, g.arg_attrs):
            if "param" in at and at["param"] not in g.constants:
                g.constants[at["param"]] = fake_data(at["param"], a.shape)
        return g

    def lookup(self, env):
        k, v, line = self.take()
        if k != "value":
            raise ParseError(f"line {line}: expected a value, got {v!r}")
        if v not in env:
            raise ParseError(f"line {line}: use of undefined value {v}")
        return env[v]

    def node(self, g, env):
        vname = self.need(kind="value")
        self.need("=")
        op = self.need(kind="ident")
        operands = []
        if self.tok[0] == "value":
            operands.append(self.lookup(env))
            while self.maybe(","):
                operands.append(self.lookup(env))
        attrs = self.attr_dict()
        self.need(":")
        t = self.tensor_type()
        node = Node(op, operands, attrs, t)
        g.nodes.append(node)
        if op == "const" and "name" in attrs and attrs["name"] not in g.constants:
            g.constants[attrs["name"]] = fake_data(attrs["name"], t.shape)
        env[vname] = node.out


def parse(text: str) -> Graph:
    from kiln.ir.core import verify

    g = _Reader(text).graph()
    verify(g)
    return g
