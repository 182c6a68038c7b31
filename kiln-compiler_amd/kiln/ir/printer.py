"""Text form of a Graph (Kiln's format, so FileCheck fixtures written for
Kiln hold here too)::

    graph @forward(%arg0: f32[2, 4]) -> (f32[2, 8]) attributes {arena_bytes = 0} {
      kernel @k0 matmul
      %0 = const {name = "fc.weight"} : f32[4, 8]
      %1 = matmul %arg0, %0 {kernel = "k0"} : f32[2, 8]
      return %1
    }

Arguments print as ``%arg<i>``, node results as ``%<i>`` in program order;
attribute values are ints, floats (Python ``repr``), booleans, quoted
strings with backslash escapes, lists and nested ``{key = value}`` maps.
"""

from __future__ import annotations


def format_attr(value) -> str:
    if value is True or value is False:
        return "true" if value else "false"
    if isinstance(value, (int, float)):
        return repr(value)
    if isinstance(value, str):
        return '"' + value.replace("\\", "\\\\").replace('"', '\\"') + '"'
    if isinstance(value, (list, tuple)):
        return "[" + ", ".join(map(format_attr, value)) + "]"
    if isinstance(value, dict):
        return format_attrs(value)
    raise TypeError(f"cannot print attribute value {value!r}")


def format_attrs(attrs: dict) -> str:
    """``{k = v, ...}``, or "" for no attributes."""
    if not attrs:
        return ""
    return "{" + ", ".join(f"{key} = {format_attr(v)}" for key, v in attrs.items()) + "}"


def _with_attrs(text: str, attrs: dict) -> str:
    return f"{text} {format_attrs(attrs)}" if attrs else text


def print_graph(graph) -> str:
    names = {}
    for i, arg in enumerate(graph.args):
        names[arg] = f"%arg{i}"
    for i, node in enumerate(graph.nodes):
        names[node.out] = f"%{i}"

    def name_of(v):
        return names.get(v, "%<undefined>")

    signature = ", ".join(_with_attrs(f"{name_of(a)}: {a.type}", attrs)
                          for a, attrs in zip(graph.args, graph.arg_attrs))
    returns = ", ".join(str(v.type) for v in graph.results)
    header = f"graph @{graph.name}({signature}) -> ({returns})"
    if graph.attrs:
        header += " attributes " + format_attrs(graph.attrs)
    lines = [header + " {"]
    lines += ["  " + _with_attrs(f"kernel @{k.name} {k.kind}", k.attrs) for k in graph.kernels]
    for node in graph.nodes:
        body = f"{name_of(node.out)} = {node.op}"
        if node.inputs:
            body += " " + ", ".join(map(name_of, node.inputs))
        lines.append(f"  {_with_attrs(body, node.attrs)} : {node.out.type}")
    lines.append("  return " + ", ".join(map(name_of, graph.results)))
    lines.append("}")
    return "\n".join(lines)
