"""Device side of one compiled graph: its buffers and the execution of its plan.

The counterpart of the reference's GPUExecutable (kiln/gpu/runtime.py:135-217).
At construction, once:

  * the plan's descriptors go to the library, which validates them and
    prepares every kernel's arguments (``kh_plan_create``);
  * the arena (every intermediate, at the memory plan's offsets) is one torch
    allocation, the constants are uploaded (or first derived on the host:
    bf16 weight copies, K-contiguous GEMV weights), a workspace is allocated
    only if some launch splits K, and the library borrows all of it
    (``kh_plan_bind``).

A call copies the inputs into static buffers, replays the plan's hipGraph
(captured at the first call) and returns clones of the static outputs -
Kiln's calling convention - or, with graphs off, runs the plan on fresh
output tensors in one ctypes call. Calls share the arena: not reentrant.
"""

from __future__ import annotations

import numpy as np
import torch

from kiln.hip import bf16
from kiln.hip import lib as kl

MiB = 2**20


def device() -> torch.device:
    """The GPU this process compiles for (PyTorch-ROCm calls it "cuda")."""
    if not torch.cuda.is_available():
        raise RuntimeError("Kiln's GPU backend needs a ROCm GPU (MI355X / gfx950); none is visible")
    return torch.device("cuda", torch.cuda.current_device())


_ready_devices = set()


def init_device(dev: torch.device):
    """kh_init once per device: checks it is a gfx950 and caches its facts."""
    index = 0 if dev.index is None else dev.index
    if index not in _ready_devices:
        kl.check(kl.load().kh_init(index), "kh_init")
        _ready_devices.add(index)


def check_memory(dev, needed_bytes, what):
    """MemoryError, before anything is allocated, if the device cannot hold
    ``needed_bytes`` (the reference's guard, kiln/gpu/runtime.py:82-90)."""
    if dev.type != "cuda":
        return
    free, total = torch.cuda.mem_get_info(dev)
    if needed_bytes <= free:
        return
    raise MemoryError(f"{what} need {needed_bytes / MiB:.1f} MiB on {dev}, which has only "
                      f"{free / MiB:.1f} MiB free of {total / MiB:.1f} MiB; free GPU memory (other processes?) "
                      f"or compile for fewer tokens")


def current_stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


class _ReplayTimer:
    """``calls`` back-to-back invocations of ``fn`` recorded once into a torch
    CUDA graph; each timed round is one replay between two events."""

    def __init__(self, fn, calls: int):
        here = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(here)
        with torch.cuda.stream(side):
            for _ in range(3):   # first-call work (allocations, caches) stays out of the graph
                fn()
        here.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for _ in range(calls):
                fn()
        self.calls = calls

    def seconds_per_call(self, rounds: int) -> float:
        self.graph.replay()
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(rounds)]
        for start, stop in marks:
            start.record()
            self.graph.replay()
            stop.record()
        torch.cuda.synchronize()
        return min(a.elapsed_time(b) for a, b in marks) * 1e-3 / self.calls


def kernel_seconds(fn, repeats=20, rounds=5) -> float:
    """GPU seconds per call of ``fn`` (any sequence of GPU work): the fastest
    of ``rounds`` replays of a graph of ``repeats`` calls, per call - the
    timing method behind the reference's published kernel numbers
    (kiln/gpu/runtime.py:93-132). Plans are timed natively instead
    (``kl.Plan.time``)."""
    return _ReplayTimer(fn, repeats).seconds_per_call(rounds)


def nk_copy(data: np.ndarray, offset: int, strides, batch: int, k: int, n: int) -> np.ndarray:
    """The fp32 [batch][N][K] copy (values unchanged, K contiguous) of the
    [batch, K, N] view (element offset, strides over (b, k, n)) of a constant:
    the layout of the K-contiguous GEMV kernel."""
    flat = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    sb, sk, sn = (int(s) for s in strides)
    idx = (offset + np.arange(batch)[:, None, None] * sb + np.arange(n)[None, :, None] * sn
           + np.arange(k)[None, None, :] * sk)
    return np.ascontiguousarray(flat[idx])


def host_constant(program, constants: dict, name: str) -> np.ndarray:
    """Host array for const slot ``name``: the fp32 constant itself, or the
    copy the lowering asked to derive from one (``program.derived``)."""
    recipe = program.derived.get(name)
    if recipe is None:
        return np.ascontiguousarray(constants[name], np.float32)
    src, offset, strides, batch, k, n = recipe[:6]
    if "@nk:" in name:
        return nk_copy(constants[src], offset, strides, batch, k, n)
    if "@nkg:" in name or "@lnc:" in name or "@lng:" in name:
        # a LayerNorm folded into the small-M GEMM that follows it: the
        # [batch][N][K] weight copy with every row scaled by gamma (one fp32
        # product per element), that copy's column sums, or beta . W per
        # column (sums in float64)
        vname, voff, vstride = recipe[6]
        w = nk_copy(constants[src], offset, strides, batch, k, n)
        vec = (np.ascontiguousarray(constants[vname], np.float32).reshape(-1)[voff + np.arange(k) * vstride]
               if vname else None)
        scaled = w if vec is None else w * vec[None, None, :]
        if "@nkg:" in name:
            return np.ascontiguousarray(scaled, dtype=np.float32)
        if "@lng:" in name:
            return np.ascontiguousarray(scaled.astype(np.float64).sum(-1).astype(np.float32))
        return np.ascontiguousarray((w.astype(np.float64) @ vec.astype(np.float64)).astype(np.float32))
    make = bf16.weight_copy_x3 if "@bf16x3:" in name else bf16.weight_copy
    return make(constants[src], offset, strides, batch, k, n).view(np.int16)


class HIPExecutable:
    """One compiled graph on one MI355X. Not reentrant."""

    def __init__(self, program, arena_bytes, constants, input_shapes, output_shapes, cuda_graphs=True,
                 debug=False, source_path=None):
        self.device = device()
        init_device(self.device)
        self.program = program
        self.source_path = source_path
        self.input_shapes = [tuple(s) for s in input_shapes]
        self.output_shapes = [tuple(s) for s in output_shapes]
        self.kernel_names = [launch.name for launch in program.launches]
        self.use_cuda_graphs = bool(cuda_graphs)
        self.debug = debug

        self.plan = kl.Plan([launch.desc for launch in program.launches])
        host = [host_constant(program, constants, name) for name in program.consts]
        self.weight_bytes = sum(int(h.nbytes) for h in host)
        self.arena_bytes = arena_bytes
        ws = self.plan.workspace_bytes
        outs = 4 * sum(int(np.prod(s)) for s in self.output_shapes)
        check_memory(self.device, arena_bytes + self.weight_bytes + ws + outs,
                     f"the arena ({arena_bytes / MiB:.1f} MiB), weights ({self.weight_bytes / MiB:.1f} MiB), "
                     f"split-K workspace ({ws / MiB:.1f} MiB) and outputs")
        self.arena = torch.empty(max(arena_bytes, 256), dtype=torch.uint8, device=self.device)
        # every split-K launch writes all the partials it reads: no clearing
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=self.device) if ws else None
        self.constants = [torch.from_numpy(h).to(self.device) for h in host]
        self.plan.bind([c.data_ptr() for c in self.constants], self.arena.data_ptr(),
                       self.workspace.data_ptr() if ws else None, ws)
        self.guards = None
        if debug:
            # launch by launch, NaN poison and canaries (kiln/hip/debug.py)
            from kiln.api import DEBUG_GUARD_BYTES
            from kiln.hip.debug import ArenaGuards, torch_ops

            self.guards = ArenaGuards(program, DEBUG_GUARD_BYTES)
            words = self.arena[: self.arena.numel() // 4 * 4].view(torch.int32)
            if self.guards.words_needed() > words.numel():
                raise RuntimeError("debug: the arena has no room for its buffers' guards (stale plan?)")
            self._guard_ops = torch_ops(words)
            self.arena.view(torch.float32)[: self.arena.numel() // 4].fill_(float("nan"))
        self._static = None   # (inputs, outputs) the hipGraph was captured over
        # with hipGraphs on, calls take graph replay (inputs copied in, outputs
        # cloned out) or launch the plan straight on the caller's tensors,
        # whichever measured faster at the first call: replay wins when a plan
        # has many short launches (the 12-layer decode: 0.265 against 0.285 ms),
        # direct launches when the copies cost more than the launches save (a
        # GPT-2 block, T = 128: 0.051 against 0.063 ms). Both run the same
        # kernels in the same order, so results are bit for bit the same.
        self.mode = None      # "graph" | "direct" once chosen
        # persistent GEMV chains bound on the GPU: a wait inside one that gives
        # up leaves NaN in every output computed from it and is counted; the
        # count is read (one device synchronisation) after the first call and
        # after every call in debug mode
        self.has_chains = any(active for _, _, active in self.plan.chains())
        self._chain_timeouts = 0
        self._chain_checked = False

    # -- inputs ---------------------------------------------------------------------------

    def _prepare(self, inputs):
        """Inputs as contiguous fp32 tensors on this device, shapes checked."""
        if len(inputs) != len(self.input_shapes):
            raise TypeError(f"expected {len(self.input_shapes)} inputs, got {len(inputs)}")
        ready = []
        for i, (t, shape) in enumerate(zip(inputs, self.input_shapes)):
            if tuple(t.shape) != shape:
                raise ValueError(f"Kiln was compiled for input shape {shape}, got {tuple(t.shape)} (input {i})")
            if t.device != self.device or t.dtype != torch.float32 or not t.is_contiguous():
                t = t.detach().to(device=self.device, dtype=torch.float32).contiguous()
            if t.data_ptr() % 16:   # kernels read rows as 16-byte pieces
                t = t.clone()
            ready.append(t)
        return ready

    # -- running -------------------------------------------------------------------------------

    def run_into(self, inputs, outputs):
        """One plan run on caller buffers (device, fp32, contiguous)."""
        ins, outs = [t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs]
        if self.guards is None:
            self.plan.run(ins, outs, current_stream_handle())
            return
        fill, differs = self._guard_ops
        for i in range(len(self.kernel_names)):
            self.guards.before(i, fill)
            self.plan.run_one(i, ins, outs, current_stream_handle())
            torch.cuda.synchronize()
            self.guards.after(i, differs)

    def _graph_buffers(self):
        if self._static is None:
            ins = [torch.zeros(s, device=self.device) for s in self.input_shapes]
            outs = [torch.empty(s, device=self.device) for s in self.output_shapes]
            torch.cuda.synchronize()
            self.plan.capture([t.data_ptr() for t in ins], [t.data_ptr() for t in outs])
            self._static = (ins, outs)
        return self._static

    @property
    def captured(self) -> bool:
        return self._static is not None

    def replay_only(self):
        """Replay the captured graph on its static buffers (benchmarks)."""
        self._graph_buffers()
        self.plan.replay(current_stream_handle())

    def _direct(self, inputs):
        outputs = [torch.empty(s, device=self.device) for s in self.output_shapes]
        self.run_into(inputs, outputs)
        return outputs

    def _replay(self, inputs):
        static_in, static_out = self._graph_buffers()
        for dst, src in zip(static_in, inputs):
            dst.copy_(src)
        self.plan.replay(current_stream_handle())
        if self.debug:
            torch.cuda.synchronize()
        return [t.clone() for t in static_out]

    def _choose_mode(self, inputs, rounds=5, calls=4):
        """Time both call paths, interleaved (so clock changes hit both alike),
        best round of `calls` calls each; replay unless direct launches win."""
        self._graph_buffers()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = {"graph": float("inf"), "direct": float("inf")}
        paths = {"graph": self._replay, "direct": self._direct}
        for fn in paths.values():
            fn(inputs)
        for _ in range(rounds):
            for name, fn in paths.items():
                start.record()
                for _ in range(calls):
                    fn(inputs)
                stop.record()
                stop.synchronize()
                best[name] = min(best[name], start.elapsed_time(stop))
        return "direct" if best["direct"] < best["graph"] else "graph"

    def check_chains(self):
        """RuntimeError if a wait inside one of the plan's persistent GEMV
        chains gave up since the last check (its outputs are NaN-poisoned)."""
        if not self.has_chains:
            return
        count = self.plan.chain_timeouts()
        new, self._chain_timeouts = count - self._chain_timeouts, count
        if new:
            raise RuntimeError(f"a persistent GEMV chain gave up {new} wait(s) (another stream's or process's "
                               f"work kept its workgroups from running together?); the outputs of this call are "
                               f"NaN from the stage that gave up on: compile with gemv_chains=False")

    def __call__(self, *inputs):
        inputs = self._prepare(inputs)
        capturing = torch.cuda.is_current_stream_capturing()
        if not self.use_cuda_graphs or capturing or self.debug:
            out = self._direct(inputs)   # also inside a caller's own stream capture; debug runs launch by launch
        else:
            if self.mode is None:
                self.mode = self._choose_mode(inputs)
            out = self._direct(inputs) if self.mode == "direct" else self._replay(inputs)
        if self.has_chains and not capturing and (self.debug or not self._chain_checked):
            self._chain_checked = True
            self.check_chains()
        return out

    def profile(self, *inputs, iters=20):
        """[(launch name, GPU ms per launch)], each launch timed natively."""
        inputs = self._prepare(inputs)
        outputs = [torch.empty(s, device=self.device) for s in self.output_shapes]
        ins, outs = [t.data_ptr() for t in inputs], [t.data_ptr() for t in outputs]
        self.run_into(inputs, outputs)
        stream = current_stream_handle()
        return [(name, 1e3 * self.plan.time(ins, outs, stream, index=i, repeats=iters, rounds=3))
                for i, name in enumerate(self.kernel_names)]
