"""``torch.compile(model, backend=kiln.backend, dynamic=False)`` on the MI355X.

Kiln's Dynamo bridge contract (the reference's kiln/backend.py:31-54): the
graphs TorchDynamo captures are traced to ATen by aot_autograd, which also
lifts the parameters into graph inputs; each forward graph is imported
(``import_fx``) and built by ``compile_graph``. The reference bridge builds
for the CPU; this one builds for the GPU.

Dynamo does not say which inputs are weights, so nothing is frozen: weights
stay runtime inputs in their own layout (a transposed view reaches the GEMM as
a strided operand) and in-place updates to them are seen by later calls. For
deployment, ``kiln.compile`` exports and freezes the model instead
(pre-transposed constants, bf16 weight copies on request).

A graph is built only when every input is a tensor on the GPU. Anything else
(CPU inputs, symbolic sizes, an op without a translation) runs as Dynamo
captured it, in eager PyTorch, after a warning, and counts in
``stats["fallback"]``; with ``KILN_STRICT=1`` it raises instead.
"""

from __future__ import annotations

import os
import warnings

import torch
from torch._dynamo.backends.common import aot_autograd
from torch._subclasses.fake_tensor import unset_fake_temporarily

stats = {"compiled": 0, "fallback": 0}


class KilnForwardCompiler:
    """aot_autograd's forward compiler: returns a callable for each graph."""

    def __init__(self, counters: dict):
        self.counters = counters

    @staticmethod
    def strict() -> bool:
        return os.environ.get("KILN_STRICT", "0") not in ("", "0", "false", "False")

    @staticmethod
    def check_inputs(example_inputs):
        from kiln.frontend.fx_import import Unsupported

        if not all(isinstance(t, torch.Tensor) for t in example_inputs):
            raise Unsupported("non-tensor graph inputs (symbolic shapes?)")
        if not all(t.device.type == "cuda" for t in example_inputs):
            raise Unsupported("this build of Kiln compiles for the MI355X GPU only; graph inputs are not all on "
                              "the CUDA device")

    def build(self, gm: torch.fx.GraphModule, example_inputs):
        from kiln.api import Options, compile_graph
        from kiln.frontend.fx_import import import_fx

        self.check_inputs(example_inputs)
        graph = import_fx(gm)
        # called under the tracer's fake-tensor mode: the executable's arena,
        # constants and plan need real device memory
        with unset_fake_temporarily():
            exe, _ = compile_graph(graph, Options(device="cuda", freeze=False))
        return exe

    def __call__(self, gm: torch.fx.GraphModule, example_inputs):
        try:
            exe = self.build(gm, example_inputs)
        except NotImplementedError as why:
            if self.strict():
                raise
            warnings.warn(f"Kiln: falling back to eager PyTorch ({why})")
            self.counters["fallback"] += 1
            return gm.forward
        self.counters["compiled"] += 1
        return lambda *args: exe(*args)


kiln_compiler = KilnForwardCompiler(stats)
backend = aot_autograd(fw_compiler=kiln_compiler)
