"""Textual form of the Kiln IR (same format as the reference's
kiln/ir/printer.py:1-79, so FileCheck expectations written against it hold):

    graph @forward(%arg0: f32[2, 4]) -> (f32[2, 8]) attributes {arena_bytes = 0} {
      kernel @k0 matmul
      %0 = const {name = "fc.weight"} : f32[4, 8]
      %1 = matmul %arg0, %0 {kernel = "k0"} : f32[2, 8]
      return %1
    }
"""

from __future__ import annotations


def format_attr(v) -> str:
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return repr(v)
    if isinstance(v, str):
        escaped = v.replace("\\", "\\\\").replace('"', '\\"')
        return f'"{escaped}"'
    if isinstance(v, (list, tuple)):
        return "[%s]" % ", ".join(format_attr(x) for x in v)
    if isinstance(v, dict):
        return format_attrs(v)
    raise TypeError(f"cannot print attribute value {v!r}")


def format_attrs(attrs: dict) -> str:
    if not attrs:
        return ""
    return "{%s}" % ", ".join(f"{k} = {format_attr(v)}" for k, v in attrs.items())


def print_graph(graph) -> str:
    name = {a: f"%arg{i}" for i, a in enumerate(graph.args)}
    name.update({n.out: f"%{i}" for i, n in enumerate(graph.nodes)})
    ref = lambda v: name.get(v, "%<undefined>")

    params = []
    for a, at in zip(graph.args, graph.arg_attrs):
        params.append(f"{ref(a)}: {a.type}" + (f" {format_attrs(at)}" if at else ""))
    head = "graph @%s(%s) -> (%s)" % (graph.name, ", ".join(params),
                                      ", ".join(str(r.type) for r in graph.results))
    if graph.attrs:
        head += " attributes " + format_attrs(graph.attrs)
    out = [head + " {"]
    for k in graph.kernels:
        out.append(f"  kernel @{k.name} {k.kind}" + (f" {format_attrs(k.attrs)}" if k.attrs else ""))
    for n in graph.nodes:
        text = f"  {ref(n.out)} = {n.op}"
        if n.inputs:
            text += " " + ", ".join(ref(v) for v in n.inputs)
        if n.attrs:
            text += " " + format_attrs(n.attrs)
        out.append(f"{text} : {n.out.type}")
    out.append("  return " + ", ".join(ref(v) for v in graph.results))
    out.append("}")
    return "\n".join(out)
