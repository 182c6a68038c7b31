"""HIP runtime: own the device buffers of a compiled graph and run its plan.

Replaces the reference's GPUExecutable (kiln/gpu/runtime.py:135-217).
Everything static is set up once:

  * the arena, one torch uint8 allocation (one hipMalloc) holding every
    intermediate at the memory plan's offsets;
  * the frozen weights, uploaded once;
  * a workspace for split-K partial tiles (every split-K launch writes all
    the partials it reads back, so it needs no initialisation);
  * the plan: every launch validated and prepared in C++ (kh_plan_create).

A call either runs the plan directly (one ctypes call for all launches) or,
with graphs on (the default), replays a hipGraph captured over static
input/output buffers: copy inputs in, replay, clone outputs out - the same
contract as the reference's CUDA-graph path (runtime.py:191-214).

Not reentrant: calls share one arena (as in the reference, runtime.py:136).
"""

from __future__ import annotations

import hashlib
import os
from pathlib import Path

import numpy as np
import torch

from kiln.hip import bf16
from kiln.hip import lib as kl


def device() -> torch.device:
    """The HIP device Kiln's GPU backend runs on (PyTorch-ROCm's "cuda")."""
    if not torch.cuda.is_available():
        raise RuntimeError("Kiln's GPU backend needs a ROCm GPU (MI355X / gfx950); none is visible")
    return torch.device("cuda", torch.cuda.current_device())


_initialised = set()


def init_device(dev: torch.device):
    if dev.index in _initialised:
        return
    lib = kl.load()
    kl.check(lib.kh_init(dev.index if dev.index is not None else 0), "kh_init")
    _initialised.add(dev.index)


def cache_dir() -> Path:
    base = os.environ.get("KILN_CACHE_DIR") or os.path.join(Path.home(), ".cache", "kiln")
    return Path(base) / "hip"


def write_source(text: str) -> Path:
    """Store the plan listing content-addressed, crash-safe (tmp + fsync +
    replace), as the reference does for its Triton source (runtime.py:58-79)."""
    digest = hashlib.sha256(text.encode()).hexdigest()[:16]
    path = cache_dir() / f"plan_{digest}.txt"
    path.parent.mkdir(parents=True, exist_ok=True)
    try:
        intact = path.read_text() == text
    except OSError:
        intact = False
    if not intact:
        tmp = path.with_suffix(f".{os.getpid()}.tmp")
        with open(tmp, "w") as f:
            f.write(text)
            f.flush()
            os.fsync(f.fileno())
        tmp.replace(path)
    return path


def check_memory(dev, needed_bytes, what):
    """Raise a clear MemoryError before allocating (reference runtime.py:82-90)."""
    if dev.type != "cuda":
        return
    free, total = torch.cuda.mem_get_info(dev)
    if needed_bytes > free:
        mib = lambda b: f"{b / 2**20:.1f} MiB"
        raise MemoryError(f"Kiln needs {mib(needed_bytes)} of GPU memory for {what}, but only "
                          f"{mib(free)} of {mib(total)} is free (other processes may be using the GPU). "
                          f"Try a smaller batch or sequence length, or free GPU memory.")


def current_stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def kernel_seconds(fn, repeats=20, rounds=5):
    """GPU time per call of ``fn``: ``repeats`` calls captured in one
    torch.cuda graph, the replay timed with events, best of ``rounds``
    (the reference's method, runtime.py:93-132)."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(repeats):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(rounds):
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        best = min(best, start.elapsed_time(end) / 1e3 / repeats)
    return best


def nk_copy(data: np.ndarray, offset: int, strides, batch: int, k: int, n: int) -> np.ndarray:
    """The fp32 [batch][N][K] copy (values unchanged, K contiguous) of the
    [batch, K, N] view (element offset, strides over (b, k, n)) of a constant:
    the layout of the K-contiguous GEMV kernel."""
    flat = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    sb, sk, sn = (int(s) for s in strides)
    idx = (offset + np.arange(batch)[:, None, None] * sb + np.arange(n)[None, :, None] * sn
           + np.arange(k)[None, None, :] * sk)
    return np.ascontiguousarray(flat[idx])


class HIPExecutable:
    """Runs one compiled graph on an MI355X. Not reentrant."""

    def __init__(self, program, arena_bytes, constants, input_shapes, output_shapes, cuda_graphs=True,
                 debug=False):
        self.device = device()
        init_device(self.device)
        self.program = program
        self.source_path = write_source(program.source)
        self.input_shapes = [tuple(s) for s in input_shapes]
        self.output_shapes = [tuple(s) for s in output_shapes]
        self.kernel_names = [l.name for l in program.launches]
        self.debug = debug

        self.plan = kl.Plan([l.desc for l in program.launches])
        host_consts = [self._host_constant(program, constants, n) for n in program.consts]
        const_bytes = sum(int(c.nbytes) for c in host_consts)
        out_bytes = sum(4 * int(np.prod(s)) for s in self.output_shapes)
        ws_bytes = self.plan.workspace_bytes
        check_memory(self.device, arena_bytes + const_bytes + out_bytes + ws_bytes,
                     f"the arena ({arena_bytes / 2**20:.1f} MiB), weights ({const_bytes / 2**20:.1f} MiB), "
                     f"workspace ({ws_bytes / 2**20:.1f} MiB) and outputs")
        self.arena = torch.empty(max(arena_bytes, 256), dtype=torch.uint8, device=self.device)
        self.workspace = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=self.device)
        self.constants = [torch.from_numpy(c).to(self.device) for c in host_consts]
        self.arena_bytes = arena_bytes
        self.weight_bytes = const_bytes
        self.plan.bind([t.data_ptr() for t in self.constants], self.arena.data_ptr(),
                       self.workspace.data_ptr(), self.workspace.numel())
        if debug:
            self.arena.view(torch.float32)[: self.arena.numel() // 4].fill_(float("nan"))
        self.use_cuda_graphs = bool(cuda_graphs)
        self.captured = False

    @staticmethod
    def _host_constant(program, constants, name):
        """Host array of const slot `name`: the fp32 constant, or a copy the
        lowering derived from one (bf16 GEMM weights, as int16 bit patterns;
        fp32 [batch][N][K] GEMV weights)."""
        if name in program.derived:
            src, offset, strides, batch, k, n = program.derived[name]
            if "@nk:" in name:
                return nk_copy(constants[src], offset, strides, batch, k, n)
            copy = bf16.weight_copy_x3 if "@bf16x3:" in name else bf16.weight_copy
            return copy(constants[src], offset, strides, batch, k, n).view(np.int16)
        return np.ascontiguousarray(constants[name], np.float32)

    # -- launching ------------------------------------------------------------------

    def _prepare(self, inputs):
        if len(inputs) != len(self.input_shapes):
            raise TypeError(f"expected {len(self.input_shapes)} inputs, got {len(inputs)}")
        out = []
        for t, shape in zip(inputs, self.input_shapes):
            if tuple(t.shape) != shape:
                raise ValueError(f"Kiln was compiled for input shape {shape}, got {tuple(t.shape)}")
            if t.device != self.device or t.dtype != torch.float32 or not t.is_contiguous():
                t = t.detach().to(self.device, torch.float32).contiguous()
            out.append(t)
        return out

    def run_into(self, inputs, outputs):
        """Run the plan on caller buffers (device, fp32, contiguous)."""
        self.plan.run([t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs], current_stream_handle())
        if self.debug:
            torch.cuda.synchronize()

    def _capture(self):
        self.static_inputs = [torch.zeros(s, device=self.device) for s in self.input_shapes]
        self.static_outputs = [torch.empty(s, device=self.device) for s in self.output_shapes]
        torch.cuda.synchronize()
        self.plan.capture([t.data_ptr() for t in self.static_inputs], [t.data_ptr() for t in self.static_outputs])
        self.captured = True

    def __call__(self, *inputs):
        inputs = self._prepare(inputs)
        if self.use_cuda_graphs:
            if not self.captured:
                self._capture()
            for static, t in zip(self.static_inputs, inputs):
                static.copy_(t)
            self.plan.replay(current_stream_handle())
            return [o.clone() for o in self.static_outputs]
        outputs = [torch.empty(s, device=self.device) for s in self.output_shapes]
        self.run_into(inputs, outputs)
        return outputs

    def replay_only(self):
        """Replay the captured graph on the static buffers (benchmarks)."""
        if not self.captured:
            self._capture()
        self.plan.replay(current_stream_handle())

    def profile(self, *inputs, iters=20):
        """Per-launch GPU time in ms: [(launch name, ms)]."""
        inputs = self._prepare(inputs)
        outputs = [torch.empty(s, device=self.device) for s in self.output_shapes]
        ins, outs = [t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs]
        self.run_into(inputs, outputs)
        times = []
        for i, l in enumerate(self.program.launches):
            fn = lambda i=i: self.plan.run_one(i, ins, outs, current_stream_handle())
            times.append((l.name, kernel_seconds(fn, repeats=iters, rounds=3) * 1e3))
        return times
