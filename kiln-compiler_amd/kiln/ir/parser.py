"""Reader for the text form that kiln/ir/printer.py writes (Kiln's grammar,
the reference's kiln/ir/parser.py:17-234)::

    graph   := 'graph' @name '(' [arg {',' arg}] ')' '->' '(' [type {',' type}] ')'
               ['attributes' attrs] '{' {kernel} {node} 'return' [%v {',' %v}] '}'
    arg     := %name ':' type [attrs]
    kernel  := 'kernel' @name kind [attrs]
    node    := %name '=' op [%v {',' %v}] [attrs] ':' type
    type    := dtype '[' [int {',' int}] ']'
    attrs   := '{' [key '=' value {',' key '=' value}] '}'

``//`` starts a comment. A ``param`` argument or named ``const`` whose data
is not supplied gets N(0, 1) * 0.1 data drawn from
``numpy.random.default_rng(zlib.crc32(name))``: the rule Kiln's own parser
uses (reference parser.py:225-227), so hand-written IR holds the same numbers
in both.

This reader is a character scanner feeding a recursive-descent parser.
"""

from __future__ import annotations

import zlib

import numpy as np

from kiln.ir.core import Graph, Kernel, Node, TensorType


class ParseError(ValueError):
    pass


def fake_data(name: str, shape) -> np.ndarray:
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    return rng.standard_normal(shape).astype(np.float32) * 0.1


_PUNCT = set("{}()[],:=")
_NAME_CHARS = set("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789_.")


class _Token:
    __slots__ = ("kind", "text", "line")

    def __init__(self, kind, text, line):
        self.kind, self.text, self.line = kind, text, line


def _scan(text: str) -> list:
    """Tokens: value (%x), symbol (@x), string, number, ident, '->' and the
    single punctuation characters; ends with an 'eof' token."""
    out, i, line, n = [], 0, 1, len(text)
    while i < n:
        c = text[i]
        if c == "\n":
            line += 1
            i += 1
        elif c.isspace():
            i += 1
        elif text.startswith("//", i):
            while i < n and text[i] != "\n":
                i += 1
        elif c in "%@":
            j = i + 1
            while j < n and text[j] in _NAME_CHARS:
                j += 1
            if j == i + 1:
                raise ParseError(f"line {line}: '{c}' without a name")
            out.append(_Token("value" if c == "%" else "symbol", text[i:j], line))
            i = j
        elif c == '"':
            j = i + 1
            while j < n and text[j] != '"':
                j += 2 if text[j] == "\\" else 1
            if j >= n:
                raise ParseError(f"line {line}: unterminated string")
            out.append(_Token("string", text[i:j + 1], line))
            i = j + 1
        elif text.startswith("->", i):
            out.append(_Token("arrow", "->", line))
            i += 2
        elif c in _PUNCT:
            out.append(_Token("punct", c, line))
            i += 1
        elif c.isdigit() or c in "+-" or c.isalpha() or c == "_":
            j = i + 1
            while j < n and (text[j] in _NAME_CHARS or (text[j] in "+-" and text[j - 1] in "eE")):
                j += 1
            word = text[i:j]
            out.append(_Token(_classify(word, line), word, line))
            i = j
        else:
            raise ParseError(f"line {line}: unexpected character {c!r}")
    out.append(_Token("eof", None, line))
    return out


def _classify(word: str, line: int) -> str:
    body = word.lstrip("+-")
    if body in ("inf", "nan"):
        return "number"
    if body[:1].isdigit():
        try:
            float(word)
        except ValueError:
            raise ParseError(f"line {line}: bad number {word!r}") from None
        return "number"
    if word[0] in "+-":
        raise ParseError(f"line {line}: unexpected {word!r}")
    return "ident"


def _number(word: str):
    body = word.lstrip("+-")
    if body.isdigit():
        return int(word)
    return float(word)


class _Parser:
    def __init__(self, text: str):
        self.tokens = _scan(text)
        self.i = 0

    # -- token helpers ------------------------------------------------------------------

    def peek(self) -> _Token:
        return self.tokens[self.i]

    def next(self) -> _Token:
        tok = self.tokens[self.i]
        self.i += 1
        return tok

    def fail(self, what, tok=None):
        tok = tok or self.peek()
        raise ParseError(f"line {tok.line}: expected {what}, got {tok.text!r}")

    def expect(self, text):
        tok = self.next()
        if tok.text != text or tok.kind == "string":
            self.fail(repr(text), tok)
        return tok

    def expect_kind(self, kind):
        tok = self.next()
        if tok.kind != kind:
            self.fail(kind, tok)
        return tok.text

    def accept(self, text) -> bool:
        tok = self.peek()
        if tok.text == text and tok.kind in ("punct", "arrow", "ident"):
            self.i += 1
            return True
        return False

    def sequence(self, close, item) -> list:
        """item {',' item} close (possibly empty)."""
        items = []
        if self.accept(close):
            return items
        items.append(item())
        while not self.accept(close):
            self.expect(",")
            items.append(item())
        return items

    # -- pieces ---------------------------------------------------------------------------

    def type(self) -> TensorType:
        dtype = self.expect_kind("ident")
        self.expect("[")
        dims = self.sequence("]", lambda: int(self.expect_kind("number")))
        return TensorType(tuple(dims), dtype)

    def attr_value(self):
        tok = self.next()
        if tok.kind == "number":
            return _number(tok.text)
        if tok.kind == "string":
            return tok.text[1:-1].encode("utf-8").decode("unicode_escape")
        if tok.kind == "ident" and tok.text in ("true", "false"):
            return tok.text == "true"
        if tok.text == "[":
            return self.sequence("]", self.attr_value)
        if tok.text == "{":
            self.i -= 1
            return self.attrs()
        self.fail("an attribute value", tok)

    def attrs(self) -> dict:
        out = {}
        if not self.accept("{"):
            return out

        def entry():
            key = self.expect_kind("ident")
            self.expect("=")
            out[key] = self.attr_value()

        self.sequence("}", entry)
        return out

    def operand(self, names):
        tok = self.next()
        if tok.kind != "value":
            self.fail("a value", tok)
        if tok.text not in names:
            raise ParseError(f"line {tok.line}: use of undefined value {tok.text}")
        return names[tok.text]

    def operands(self, names) -> list:
        found = []
        if self.peek().kind == "value":
            found.append(self.operand(names))
            while self.accept(","):
                found.append(self.operand(names))
        return found

    # -- the graph ---------------------------------------------------------------------------

    def graph(self) -> Graph:
        self.expect("graph")
        graph = Graph(self.expect_kind("symbol")[1:])
        names = {}

        def argument():
            label = self.expect_kind("value")
            self.expect(":")
            t = self.type()
            attrs = self.attrs()
            names[label] = graph.add_arg(t, attrs.get("param", label[1:]), **attrs)

        self.expect("(")
        self.sequence(")", argument)
        self.expect("->")
        self.expect("(")
        result_types = self.sequence(")", self.type)
        if self.accept("attributes"):
            graph.attrs = self.attrs()
        self.expect("{")
        while self.peek().text == "kernel":
            self.next()
            kname = self.expect_kind("symbol")[1:]
            kkind = self.expect_kind("ident")
            graph.kernels.append(Kernel(kname, kkind, [], self.attrs()))
        while self.peek().kind == "value":
            self.node(graph, names)
        tok = self.peek()
        if tok.text != "return":
            self.fail("a node or 'return'", tok)
        self.next()
        graph.results = self.operands(names)
        self.expect("}")
        if self.peek().kind != "eof":
            self.fail("end of input")
        if [v.type for v in graph.results] != result_types:
            raise ParseError(f"graph @{graph.name}: declared result types {[str(t) for t in result_types]} "
                             f"differ from the returned values")
        self._attach(graph)
        return graph

    def node(self, graph, names):
        label = self.expect_kind("value")
        self.expect("=")
        op = self.expect_kind("ident")
        inputs = self.operands(names)
        attrs = self.attrs()
        self.expect(":")
        node = Node(op, inputs, attrs, self.type())
        graph.nodes.append(node)
        names[label] = node.out

    @staticmethod
    def _attach(graph):
        """Give kernels their nodes and missing data its name-seeded values."""
        kernels = {k.name: k for k in graph.kernels}
        for node in graph.nodes:
            if "kernel" in node.attrs:
                owner = kernels.get(node.attrs["kernel"])
                if owner is None:
                    raise ParseError(f"node refers to undeclared kernel @{node.attrs['kernel']}")
                owner.nodes.append(node)
            if node.op == "const" and "name" in node.attrs and node.attrs["name"] not in graph.constants:
                graph.constants[node.attrs["name"]] = fake_data(node.attrs["name"], node.out.type.shape)
        for arg, attrs in zip(graph.args, graph.arg_attrs):
            if "param" in attrs and attrs["param"] not in graph.constants:
                graph.constants[attrs["param"]] = fake_data(attrs["param"], arg.type.shape)


def parse(text: str) -> Graph:
    """Parse and verify one graph."""
    from kiln.ir.core import verify

    graph = _Parser(text).graph()
    verify(graph)
    return graph
