"""Public API: ``kiln.compile(model, example_inputs, device="cuda")``.

Contract of the reference's kiln/api.py:14-276: the same ``Options`` fields
and flag overrides (unknown flag -> TypeError), the same pass pipeline
(``build_passes``), ``Report`` and ``CompiledModule``. The GPU target is this
build's MI355X HIP backend (kiln/hip); the reference's MLIR CPU backend is
not part of this build, so ``device="cpu"`` raises NotImplementedError.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from kiln.ir.core import Graph


@dataclass
class Options:
    """Which optimisations to run. Every flag can be turned off for ablations."""

    freeze: bool = True          # parameters -> constants, then constant folding
    fusion: bool = True          # multi-op kernels (otherwise one op per kernel)
    memory_plan: bool = True     # buffers share arena memory when lifetimes don't overlap
    tiling: bool = True          # CPU backend only (loop tiling); ignored on the GPU
    target: object = None        # CPU backend only
    autotune: bool = False       # choose GEMM tiles by measurement (cached on disk)
    matmul_tiles_for: object = None   # CPU backend only
    print_ir: bool = False       # print the Kiln IR after every pass
    dump_mlir: bool = False      # GPU: print the lowered HIP plan
    profile: bool = False        # keep per-launch names for CompiledModule.profile()
    device: str = "cpu"          # "cuda": the MI355X HIP backend
    allow_tf32: bool = False     # gfx950 has no TF32 MFMA: maps to the bf16x3 GEMM (~fp32-class error)
    cuda_graphs: bool = True     # GPU: replay the whole plan as one hipGraph
    gpu_matmul_config: object = None  # advanced: fn(graph, kernel) -> {"tile": id, "splitk": s}
    matmul_precision: str = "fp32"    # GPU GEMMs: "fp32" | "bf16" (bf16 inputs, fp32 accumulate) | "bf16x3"
    debug: bool = False          # GPU: NaN-poison the arena and synchronise after every plan run
    fused_attention: bool = True # GPU: scores -> softmax -> (x V) as one kernel (needs fusion)

    @classmethod
    def none(cls, **kw):
        """Every optimisation off: the baseline for ablations."""
        return cls(freeze=False, fusion=False, memory_plan=False, tiling=False, **kw)


@dataclass
class Report:
    passes: dict = field(default_factory=dict)
    timings: dict = field(default_factory=dict)
    lowering: dict = field(default_factory=dict)
    kernels: list = field(default_factory=list)
    arena_bytes: int = 0
    naive_bytes: int = 0         # arena without reuse (one slot per buffer)
    lower_bound_bytes: int = 0   # peak live bytes: no plan can be smaller
    compile_seconds: float = 0.0
    autotune: list = field(default_factory=list)

    def __str__(self):
        lines = [f"Kiln: {len(self.kernels)} kernels, compiled in {self.compile_seconds:.2f}s"]
        lines += [f"  {k}" for k in self.kernels]
        lines.append(f"  arena: {self.arena_bytes} bytes (no reuse: {self.naive_bytes}, "
                     f"lower bound: {self.lower_bound_bytes})")
        low = self.lowering
        if low.get("backend") == "hip":
            lines.append(f"  GPU: {low['launches']} HIP kernel launches ({low.get('families')}), "
                         f"hipGraph: {low['cuda_graphs']}, precision: {low.get('precision')}, "
                         f"plan: {low['source']}")
        for name, stats in self.passes.items():
            lines.append(f"  {name}: {stats}")
        for e in self.autotune:
            b, m, n, k = e["shape"]
            lines.append(f"  autotune {b}x{m}x{n}x{k} ({e['source']}): {e['default_tflops']} -> "
                         f"{e['tflops']} TFLOP/s, config {e['config']}")
        return "\n".join(lines)


def build_passes(options: Options, tuner=None):
    """The pass pipeline (reference api.py:78-95, without the CPU Schedule)."""
    from kiln.passes.buffers import BufferAssignment
    from kiln.passes.freeze import ConstantFold, FreezeParameters
    from kiln.passes.fusion import Fusion
    from kiln.passes.memory_plan import MemoryPlan
    from kiln.passes.partition import OneOpPerKernel
    from kiln.passes.simplify import CSE, DCE, Canonicalize

    passes = [Canonicalize(), CSE()]
    if options.freeze:
        passes += [FreezeParameters(), ConstantFold(), Canonicalize(), CSE()]
    passes += [DCE(), Fusion() if options.fusion else OneOpPerKernel(),
               BufferAssignment(), MemoryPlan(reuse=options.memory_plan)]
    return passes


def compile_graph(graph: Graph, options: Options | None = None):
    """Optimise a Kiln graph and build it for the device. Returns (executable, Report)."""
    options = options or Options()
    if options.device not in ("cpu", "cuda"):
        raise ValueError(f"device must be 'cpu' or 'cuda', got {options.device!r}")
    if options.device == "cpu":
        raise NotImplementedError("this build of Kiln contains only the MI355X GPU backend; "
                                  "compile with device='cuda'")
    return _compile_graph_gpu(graph, options)


def _precision(options: Options) -> str:
    if options.matmul_precision not in ("fp32", "bf16", "bf16x3"):
        raise ValueError(f"matmul_precision must be fp32, bf16 or bf16x3, got {options.matmul_precision!r}")
    if options.allow_tf32 and options.matmul_precision == "fp32":
        return "bf16x3"
    return options.matmul_precision


def _compile_graph_gpu(graph: Graph, options: Options):
    """Passes, then lowering to HIP kernel families, then the executable."""
    from kiln.hip.lib import FAMILY_NAMES
    from kiln.hip.lowering import lower_graph
    from kiln.hip.runtime import HIPExecutable
    from kiln.passes.manager import PassManager

    start = time.perf_counter()
    passes = build_passes(options)
    if options.fusion and options.fused_attention:
        from kiln.hip.attention import FuseAttention

        passes.insert(len(passes) - 1, FuseAttention())   # after buffer-assign, before memory-plan
    pm = PassManager(passes, print_after_all=options.print_ir)
    pm.run(graph)
    precision = _precision(options)
    tuner = None
    config_for = options.gpu_matmul_config
    if config_for is None and options.autotune:
        from kiln.hip.autotune import GPUAutotuner

        tuner = GPUAutotuner(precision=precision)
        config_for = tuner.config_for
    program = lower_graph(graph, precision=precision, matmul_config=config_for)
    exe = HIPExecutable(program, graph.attrs.get("arena_bytes", 0), graph.constants,
                        [a.shape for a in graph.args], [r.shape for r in graph.results],
                        cuda_graphs=options.cuda_graphs, debug=options.debug)
    if options.dump_mlir:
        print(f"// ----- lowered HIP plan ({exe.source_path}) -----\n{program.source}")
    families = {}
    for l in program.launches:
        families[FAMILY_NAMES[l.family]] = families.get(FAMILY_NAMES[l.family], 0) + 1
    report = Report(passes=pm.stats, timings=pm.timings)
    report.lowering = {"backend": "hip", "launches": len(program.launches), "source": str(exe.source_path),
                       "cuda_graphs": exe.use_cuda_graphs, "tf32": options.allow_tf32,
                       "precision": precision, "families": families}
    report.kernels = [f"{k.name} {k.kind:<11} {' '.join(n.op for n in k.nodes)}" for k in graph.kernels]
    report.arena_bytes = graph.attrs.get("arena_bytes", 0)
    plan = pm.stats.get("memory-plan", {})
    report.naive_bytes = plan.get("naive_bytes", 0)
    report.lower_bound_bytes = plan.get("lower_bound_bytes", 0)
    report.autotune = tuner.log if tuner is not None else []
    report.compile_seconds = time.perf_counter() - start
    return exe, report


class CompiledModule:
    """Callable returned by ``kiln.compile``."""

    def __init__(self, exe, report, graph, param_tensors, single_output):
        self._exe = exe
        self.report = report
        self.graph = graph
        self._params = param_tensors     # (position, tensor) for unfrozen parameters
        self._single = single_output
        self._positions = [i for i, a in enumerate(graph.arg_attrs) if "param" not in a]

    def _args(self, inputs):
        if len(inputs) != len(self._positions):
            raise TypeError(f"expected {len(self._positions)} inputs, got {len(inputs)}")
        args = [None] * len(self.graph.args)
        for pos, t in zip(self._positions, inputs):
            args[pos] = t
        for pos, t in self._params:
            args[pos] = t
        return args

    def profile(self, *inputs, iters=20):
        """Per-launch GPU times in ms: [(launch, kernel kind, ops, ms)]."""
        times = self._exe.profile(*self._args(inputs), iters=iters)
        by_name = {l.name: l for l in self._exe.program.launches}
        kinds = {k.name: k for k in self.graph.kernels}
        out = []
        for name, ms in times:
            k = kinds[by_name[name].kernel]
            out.append((name, k.kind, " ".join(n.op for n in k.nodes), ms))
        return out

    def __call__(self, *inputs):
        outs = self._exe(*self._args(inputs))
        return outs[0] if self._single else tuple(outs)


class _FnModule(torch.nn.Module):
    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, *args):
        return self.fn(*args)


def compile(model, example_inputs, options: Options | None = None, **flags) -> CompiledModule:
    """Compile a model (or function) for inference.

        compiled = kiln.compile(model, (x,), device="cuda")
        y = compiled(x)
        print(compiled.report)

    Keyword flags override fields of ``options`` (unknown flag -> TypeError).
    """
    from kiln.frontend.fx_import import import_exported

    options = options or Options()
    for key, value in flags.items():
        if not hasattr(options, key):
            raise TypeError(f"unknown option {key!r}")
        setattr(options, key, value)

    module = model if isinstance(model, torch.nn.Module) else _FnModule(model)
    was_training = module.training
    module.eval()
    try:
        with torch.no_grad():
            ep = torch.export.export(module, tuple(example_inputs)).run_decompositions()
            single = not isinstance(module(*example_inputs), (tuple, list))
    finally:
        module.train(was_training)

    graph = import_exported(ep)
    live = dict(module.named_parameters()) | dict(module.named_buffers())
    exe, report = compile_graph(graph, options)
    params = [(i, live[a["param"]].detach()) for i, a in enumerate(graph.arg_attrs) if "param" in a]
    # Unfrozen weights are runtime inputs, moved to the GPU once here; a model
    # already on the GPU shares its weight memory (and so its in-place updates).
    params = [(i, t.to(exe.device)) for i, t in params]
    return CompiledModule(exe, report, graph, params, single)
