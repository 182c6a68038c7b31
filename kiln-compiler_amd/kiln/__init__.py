"""Kiln: an inference compiler for PyTorch models, with an MI355X (gfx950) backend.

    import kiln
    compiled = kiln.compile(model, (example_input,), device="cuda")
    y = compiled(x)

    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)

The compiler front half (IR, freeze/fusion/buffer/memory-plan passes) keeps the
reference Kiln's contracts; below it, every fused kernel runs on a hand-written
HIP kernel family from libkiln_hip.so, replayed as one hipGraph.
"""

from kiln.api import CompiledModule, Options, Report, compile, compile_graph
from kiln.backend import backend, stats

__all__ = ["compile", "compile_graph", "Options", "Report", "CompiledModule", "backend", "stats"]
