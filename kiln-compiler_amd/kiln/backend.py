"""torch.compile backend for the MI355X HIP path.

    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)

Same contract as the reference bridge (kiln/backend.py:31-54): aot_autograd
traces each graph TorchDynamo captures down to ATen ops and lifts the
parameters into graph inputs; the forward graph is imported
(frontend.fx_import.import_fx) and compiled by compile_graph. Dynamo does not
say which inputs are weights, so freezing is off: weights stay runtime
inputs, read in their original layout (a transposed view feeds the GEMM as a
strided operand), and in-place updates to them are seen by later calls. For
inference deployments prefer ``kiln.compile``, which exports the model and
freezes it (pre-transposed constants, bf16 weight copies when asked).

This build compiles for the GPU only: graphs whose tensor inputs are on the
CUDA device are built for it; any other graph (CPU inputs, symbolic shapes,
an op without a lowering) falls back to eager PyTorch with a warning.

Environment variables:
    KILN_STRICT=1   raise on unsupported graphs instead of falling back to eager
"""

from __future__ import annotations

import os
import warnings

import torch
from torch._dynamo.backends.common import aot_autograd
from torch._subclasses.fake_tensor import unset_fake_temporarily

stats = {"compiled": 0, "fallback": 0}


def _strict() -> bool:
    return os.environ.get("KILN_STRICT", "0") not in ("", "0", "false", "False")


def _device_of(example_inputs) -> str:
    from kiln.frontend.fx_import import Unsupported

    tensors = [t for t in example_inputs if isinstance(t, torch.Tensor)]
    if len(tensors) != len(example_inputs):
        raise Unsupported("non-tensor graph inputs (symbolic shapes?)")
    if tensors and all(t.device.type == "cuda" for t in tensors):
        return "cuda"
    raise Unsupported("this build of Kiln compiles for the MI355X GPU only; graph inputs are not all on the "
                      "CUDA device")


def kiln_compiler(gm: torch.fx.GraphModule, example_inputs):
    """aot_autograd forward compiler: an executable for `gm`, or gm.forward."""
    from kiln.api import Options, compile_graph
    from kiln.frontend.fx_import import import_fx

    try:
        device = _device_of(example_inputs)
        graph = import_fx(gm)
        # the compiler is called inside the tracer's fake-tensor mode; the
        # executable's arena, workspace and plan need real device memory
        with unset_fake_temporarily():
            exe, _ = compile_graph(graph, Options(device=device, freeze=False))
    except NotImplementedError as err:
        if _strict():
            raise
        warnings.warn(f"Kiln: falling back to eager PyTorch ({err})")
        stats["fallback"] += 1
        return gm.forward

    stats["compiled"] += 1

    def run(*args):
        return exe(*args)

    return run


# aot_autograd traces down to ATen ops and lifts parameters into graph inputs.
backend = aot_autograd(fw_compiler=kiln_compiler)
