from kiln.ir.core import Graph, Kernel, Node, TensorType, Value, verify
from kiln.ir.ops import interpret
from kiln.ir.parser import parse

__all__ = ["Graph", "Kernel", "Node", "TensorType", "Value", "verify", "interpret", "parse"]
