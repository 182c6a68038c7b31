"""Running a compiled plan's meaning on the CPU (``KILN_HIP_INTERPRET=1``).

The counterpart of the reference's interpreter switch
(kiln/gpu/runtime.py:39-50: with ``TRITON_INTERPRET=1`` its GPU tests run the
generated kernels on the CPU). Here the library's ``kh_plan_run_host``
executes every launch of the plan, straight from its descriptors, over numpy
buffers. The whole compile path is the real one (passes, lowering, plan
creation and validation in the library); only the execution is the host
interpreter's.

It is opt-in and a test instrument: it is chosen only when the environment
asks for it, never as a fallback, and the GPU tests, ``smoke()`` and
``bench.py`` refuse to run with it set. Constants, the arena and inputs are
host arrays; the arena is filled with NaN first, so a launch that reads an
intermediate no launch wrote shows up in the result. Outputs are CPU tensors.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from kiln.hip import lib as kl
from kiln.hip.runtime import host_constant


def interpreting() -> bool:
    return os.environ.get("KILN_HIP_INTERPRET", "0") not in ("", "0", "false", "False")


def refuse(what: str):
    """For GPU measurements and GPU tests: the interpreter must not be on."""
    if interpreting():
        raise RuntimeError(f"{what} needs the GPU path; unset KILN_HIP_INTERPRET")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class HostExecutable:
    """The HIPExecutable interface over host memory."""

    def __init__(self, program, arena_bytes, constants, input_shapes, output_shapes, cuda_graphs=True,
                 debug=False, source_path=None):
        self.device = torch.device("cpu")
        self.program = program
        self.source_path = source_path
        self.input_shapes = [tuple(s) for s in input_shapes]
        self.output_shapes = [tuple(s) for s in output_shapes]
        self.kernel_names = [launch.name for launch in program.launches]
        self.use_cuda_graphs = False
        self.plan = kl.Plan([launch.desc for launch in program.launches])
        self.constants = [np.ascontiguousarray(host_constant(program, constants, name)) for name in program.consts]
        self.weight_bytes = sum(int(c.nbytes) for c in self.constants)
        self.arena_bytes = arena_bytes
        self.arena = np.full(max(arena_bytes, 256) // 4, np.nan, dtype=np.float32)
        consts = [_ptr(c) for c in self.constants]
        self.plan.bind(consts, _ptr(self.arena), None, 0)
        self.guards = None
        if debug:
            # launch by launch (one single-launch plan each), NaN poison and
            # canaries as on the device (kiln/hip/debug.py)
            from kiln.api import DEBUG_GUARD_BYTES
            from kiln.hip.debug import ArenaGuards, numpy_ops

            self.guards = ArenaGuards(program, DEBUG_GUARD_BYTES)
            if self.guards.words_needed() > self.arena.size:
                raise RuntimeError("debug: the arena has no room for its buffers' guards (stale plan?)")
            self._guard_ops = numpy_ops(self.arena.view(np.int32))
            self._single = []
            for launch in program.launches:
                one = kl.Plan([launch.desc])
                one.bind(consts, _ptr(self.arena), None, 0)
                self._single.append(one)

    def _prepare(self, inputs):
        if len(inputs) != len(self.input_shapes):
            raise TypeError(f"expected {len(self.input_shapes)} inputs, got {len(inputs)}")
        ready = []
        for i, (t, shape) in enumerate(zip(inputs, self.input_shapes)):
            if tuple(t.shape) != shape:
                raise ValueError(f"Kiln was compiled for input shape {shape}, got {tuple(t.shape)} (input {i})")
            ready.append(np.ascontiguousarray(t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else t,
                                              dtype=np.float32))
        return ready

    def __call__(self, *inputs):
        ins = self._prepare(inputs)
        outs = [np.full(s, np.nan, dtype=np.float32) for s in self.output_shapes]
        in_ptrs, out_ptrs = [_ptr(a) for a in ins], [_ptr(a) for a in outs]
        if self.guards is None:
            self.plan.run_host(in_ptrs, out_ptrs)
        else:
            fill, differs = self._guard_ops
            for i, one in enumerate(self._single):
                self.guards.before(i, fill)
                one.run_host(in_ptrs, out_ptrs)
                self.guards.after(i, differs)
        return [torch.from_numpy(o) for o in outs]
