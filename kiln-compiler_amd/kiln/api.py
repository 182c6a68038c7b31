"""``kiln.compile(model, example_inputs, device="cuda")`` and what it returns.

The interface is Kiln's (the reference's kiln/api.py:14-276): ``Options``
with the same fields and per-call flag overrides (an unknown flag is a
TypeError), ``build_passes``, ``compile_graph(graph, options) ->
(executable, Report)``, ``Report`` and ``CompiledModule``. The target is
this build's MI355X HIP backend; Kiln's MLIR CPU backend is not part of it,
so ``device="cpu"`` raises NotImplementedError.

A GPU build runs in four steps (``_GpuBuild``): the pass pipeline; the plan,
taken from the on-disk plan store when the same optimised graph was lowered
before for this device and settings (kiln/hip/plans.py), else lowered now
(kiln/hip/lowering.py, with GEMM configurations from the tuner or the
default model) and stored; the executable; the report.
"""

from __future__ import annotations

import copy
import time
from dataclasses import dataclass, field, fields

import torch

from kiln.ir.core import Graph


@dataclass
class Options:
    """What the compiler does. Every optimisation can be switched off for
    ablations; ``Options.none()`` switches them all off."""

    freeze: bool = True          # weights become constants, then constant folding
    fusion: bool = True          # multi-op kernels (else one op per kernel)
    memory_plan: bool = True     # intermediates share arena space when their lifetimes do not overlap
    tiling: bool = True          # Kiln's CPU backend only (loop tiling); no effect here
    target: object = None        # Kiln's CPU backend only
    autotune: bool = False       # measure GEMM configurations (cached on disk)
    matmul_tiles_for: object = None   # Kiln's CPU backend only
    print_ir: bool = False       # print the IR after every pass
    dump_mlir: bool = False      # print the lowered HIP plan listing
    profile: bool = False        # accepted; per-launch names are always kept for profile()
    device: str = "cpu"          # "cuda": the MI355X HIP backend
    allow_tf32: bool = False     # gfx950 has no TF32 MFMA: selects the three-pass bf16 GEMM (fp32-class error)
    cuda_graphs: bool = True     # replay the whole plan as one hipGraph
    gpu_matmul_config: object = None  # fn(graph, kernel) -> {"tile": id, "splitk": s}, overrides tuning
    matmul_precision: str = "fp32"    # GEMM inputs: "fp32" | "bf16" (fp32 accumulate) | "bf16x3"
    debug: bool = False          # launch by launch: NaN-poison each arena buffer before the launch that first
                                 # writes it, canaries between buffers checked after every launch
    fused_attention: bool = True # scores -> softmax -> (x V) as one launch (needs fusion)
    plan_cache: bool = True      # reuse plans lowered earlier for the same graph and settings
    gemv_chains: bool = False    # consecutive one-row matmuls (decode) as one persistent launch (measured
                                 # slower than launch by launch at the GPT-2 decode sizes, so opt-in)

    @classmethod
    def none(cls, **overrides):
        return cls(freeze=False, fusion=False, memory_plan=False, tiling=False, **overrides)

    def overridden(self, **flags) -> "Options":
        """A copy with ``flags`` applied; TypeError for a name that is not a field."""
        known = {f.name for f in fields(self)}
        unknown = sorted(set(flags) - known)
        if unknown:
            raise TypeError(f"unknown option {unknown[0]!r}")
        out = copy.copy(self)
        for name, value in flags.items():
            setattr(out, name, value)
        return out

    def gemm_precision(self) -> str:
        if self.matmul_precision not in ("fp32", "bf16", "bf16x3"):
            raise ValueError(f"matmul_precision must be fp32, bf16 or bf16x3, got {self.matmul_precision!r}")
        if self.allow_tf32 and self.matmul_precision == "fp32":
            return "bf16x3"
        return self.matmul_precision


@dataclass
class Report:
    passes: dict = field(default_factory=dict)     # pass name -> statistics
    timings: dict = field(default_factory=dict)    # pass name -> seconds
    lowering: dict = field(default_factory=dict)   # backend, launches, source, cuda_graphs, tf32, ...
    kernels: list = field(default_factory=list)    # "k<i> <kind> <ops>" per fused kernel
    arena_bytes: int = 0
    naive_bytes: int = 0         # one arena slot per buffer, no reuse
    lower_bound_bytes: int = 0   # peak of simultaneously live bytes: no plan is smaller
    compile_seconds: float = 0.0
    autotune: list = field(default_factory=list)

    def __str__(self):
        out = [f"Kiln: {len(self.kernels)} fused kernels, compiled in {self.compile_seconds:.2f} s"]
        out += ["  " + k for k in self.kernels]
        out.append(f"  arena {self.arena_bytes} B (without reuse {self.naive_bytes} B, "
                   f"peak live {self.lower_bound_bytes} B)")
        low = self.lowering
        if low.get("backend") == "hip":
            out.append(f"  MI355X: {low['launches']} launches {low.get('families')}, "
                       f"precision {low.get('precision')}, hipGraph {'on' if low['cuda_graphs'] else 'off'}, "
                       f"plan {low.get('plan_cache', 'lowered')}: {low['source']}")
        out += [f"  pass {name}: {stats}" for name, stats in self.passes.items()]
        for e in self.autotune:
            shape = "x".join(map(str, e["shape"]))
            out.append(f"  gemm {shape} [{e['source']}] config {e['config']}: "
                       f"{e['default_tflops']} -> {e['tflops']} TFLOP/s")
        return "\n".join(out)


def build_passes(options: Options, tuner=None) -> list:
    """Kiln's pipeline (the reference's api.py:78-95, without the CPU-only
    scheduling pass): clean-up, freezing and folding, partition into kernels,
    buffer assignment, memory planning."""
    from kiln.passes.buffers import BufferAssignment
    from kiln.passes.freeze import ConstantFold, FreezeParameters
    from kiln.passes.fusion import Fusion
    from kiln.passes.memory_plan import MemoryPlan
    from kiln.passes.partition import OneOpPerKernel
    from kiln.passes.simplify import CSE, DCE, Canonicalize

    cleanup = [Canonicalize(), CSE()]
    pipeline = list(cleanup)
    if options.freeze:
        pipeline += [FreezeParameters(), ConstantFold(), *[type(p)() for p in cleanup]]
    pipeline.append(DCE())
    pipeline.append(Fusion() if options.fusion else OneOpPerKernel())
    pipeline += [BufferAssignment(), MemoryPlan(reuse=options.memory_plan, guard=DEBUG_GUARD_BYTES if options.debug else 0)]
    return pipeline


# canary bytes after every arena buffer in debug builds (Options.debug)
DEBUG_GUARD_BYTES = 256


def compile_graph(graph: Graph, options: Options | None = None):
    """Optimise ``graph`` and build it for ``options.device``; returns
    (executable, Report)."""
    options = options or Options()
    if options.device == "cuda":
        return _GpuBuild(graph, options).run()
    if options.device == "cpu":
        raise NotImplementedError("this build of Kiln contains only the MI355X GPU backend; "
                                  "compile with device='cuda'")
    raise ValueError(f"device must be 'cpu' or 'cuda', got {options.device!r}")


def _compile_graph_gpu(graph: Graph, options: Options):
    """The GPU branch of compile_graph (the reference's api.py:142-180)."""
    return _GpuBuild(graph, options).run()


class _GpuBuild:
    def __init__(self, graph: Graph, options: Options):
        self.graph = graph
        self.options = options
        self.precision = options.gemm_precision()
        self.started = time.perf_counter()

    def optimise(self):
        from kiln.passes.manager import PassManager

        passes = build_passes(self.options)
        if self.options.fusion and self.options.fused_attention:
            from kiln.hip.attention import FuseAttention

            passes.insert(len(passes) - 1, FuseAttention())   # after buffer assignment, before the memory plan
        self.pm = PassManager(passes, print_after_all=self.options.print_ir)
        self.pm.run(self.graph)

    def config_source(self):
        """(fn(graph, kernel) -> config or None, its name for the plan key or
        None when the plans it makes cannot be keyed, the tuner or None)."""
        from kiln.hip.interpret import interpreting

        if self.options.gpu_matmul_config is not None:
            return self.options.gpu_matmul_config, None, None
        if self.options.autotune and not interpreting():   # nothing to measure on the host interpreter
            from kiln.hip.autotune import GPUAutotuner

            tuner = GPUAutotuner(precision=self.precision)
            return tuner.config_for, "autotune", tuner
        return None, "default", None

    def plan(self):
        from kiln.hip import lib as kl
        from kiln.hip import plans
        from kiln.hip.lowering import lower_graph

        config_for, source_name, tuner = self.config_source()
        key = None
        if self.options.plan_cache and source_name is not None:
            from kiln.hip import lowering

            source = source_name + "|gemv-chains" if self.options.gemv_chains else source_name
            if lowering.ATTN_QUERIES:
                source += f"|attention-q{lowering.ATTN_QUERIES}"
            key = plans.plan_key(str(self.graph), self.precision, source, kl.device_info())
            stored = plans.load(key)
            if stored is not None:
                program, log = stored
                return program, log, plans.listing_path(key), "stored"
        program = lower_graph(self.graph, precision=self.precision, matmul_config=config_for,
                              gemv_chains=self.options.gemv_chains)
        log = tuner.log if tuner is not None else []
        if key is None:   # a caller's config function: the plan cannot be keyed, only listed
            return program, log, plans.write_listing("unkeyed-" + program.digest(), program), "lowered"
        return program, log, plans.save(key, program, log), "lowered"

    def run(self):
        from kiln.hip.interpret import HostExecutable, interpreting
        from kiln.hip.lib import FAMILY_NAMES
        from kiln.hip.runtime import HIPExecutable

        self.optimise()
        program, autotune_log, listing, origin = self.plan()
        g = self.graph
        # KILN_HIP_INTERPRET=1 (tests only): the plan's meaning on the CPU
        executable = HostExecutable if interpreting() else HIPExecutable
        exe = executable(program, g.attrs.get("arena_bytes", 0), g.constants, [a.shape for a in g.args],
                            [r.shape for r in g.results], cuda_graphs=self.options.cuda_graphs,
                            debug=self.options.debug, source_path=listing)
        if self.options.dump_mlir:
            print(f"// ----- lowered HIP plan ({listing}) -----\n{program.source}")
        families = {}
        for launch in program.launches:
            name = FAMILY_NAMES[launch.family]
            families[name] = families.get(name, 0) + 1
        memory = self.pm.stats.get("memory-plan", {})
        # persistent GEMV chains the library formed: each runs as one kernel launch
        plan = getattr(exe, "plan", None)
        chains = plan.chains() if plan is not None else []
        kernel_launches = len(program.launches) - sum(n - 1 for _, n, active in chains if active)
        report = Report(
            passes=self.pm.stats, timings=self.pm.timings,
            lowering={"backend": "hip", "launches": len(program.launches), "source": str(listing),
                      "cuda_graphs": exe.use_cuda_graphs, "tf32": self.options.allow_tf32,
                      "precision": self.precision, "families": families, "plan_cache": origin,
                      "gemv_chains": [(first, n) for first, n, _ in chains], "kernel_launches": kernel_launches},
            kernels=[f"{k.name} {k.kind:<11} {' '.join(n.op for n in k.nodes)}" for k in g.kernels],
            arena_bytes=g.attrs.get("arena_bytes", 0), naive_bytes=memory.get("naive_bytes", 0),
            lower_bound_bytes=memory.get("lower_bound_bytes", 0), autotune=list(autotune_log))
        report.compile_seconds = time.perf_counter() - self.started
        return exe, report


class CompiledModule:
    """What ``kiln.compile`` returns: call it like the model."""

    def __init__(self, exe, report, graph, param_tensors, single_output):
        self._exe = exe
        self.report = report
        self.graph = graph
        self._single = single_output
        # graph argument order: runtime inputs fill the slots that are not
        # (unfrozen) parameters, which are bound to the model's own tensors
        self._bound = dict(param_tensors)
        self._free = [i for i in range(len(graph.args)) if i not in self._bound]

    def _graph_args(self, inputs):
        if len(inputs) != len(self._free):
            raise TypeError(f"expected {len(self._free)} inputs, got {len(inputs)}")
        args = [None] * len(self.graph.args)
        for slot, t in zip(self._free, inputs):
            args[slot] = t
        for slot, t in self._bound.items():
            args[slot] = t
        return args

    def __call__(self, *inputs):
        outputs = self._exe(*self._graph_args(inputs))
        return outputs[0] if self._single else tuple(outputs)

    def profile(self, *inputs, iters=20):
        """GPU time of every launch: [(launch, kernel kind, ops, ms)]."""
        launches = {launch.name: launch for launch in self._exe.program.launches}
        kernels = {k.name: k for k in self.graph.kernels}
        rows = []
        for name, ms in self._exe.profile(*self._graph_args(inputs), iters=iters):
            kernel = kernels[launches[name].kernel]
            rows.append((name, kernel.kind, " ".join(n.op for n in kernel.nodes), ms))
        return rows


class _FnModule(torch.nn.Module):
    """Lets a plain function go through torch.export."""

    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, *args):
        return self.fn(*args)


def _export(module: torch.nn.Module, example_inputs):
    """(decomposed ExportedProgram, whether the module returns one tensor).
    The module runs in eval mode for the export and gets its mode back."""
    training = module.training
    module.eval()
    try:
        with torch.no_grad():
            ep = torch.export.export(module, tuple(example_inputs)).run_decompositions()
            single = not isinstance(module(*example_inputs), (tuple, list))
    finally:
        module.train(training)
    return ep, single


def compile(model, example_inputs, options: Options | None = None, **flags) -> CompiledModule:
    """Compile ``model`` (an nn.Module or a function of tensors) for inference
    on the example inputs' shapes::

        compiled = kiln.compile(model, (x,), device="cuda")
        y = compiled(x)
        print(compiled.report)

    Keyword flags override fields of ``options``.
    """
    from kiln.frontend.fx_import import import_exported

    options = (options or Options()).overridden(**flags)
    module = model if isinstance(model, torch.nn.Module) else _FnModule(model)
    ep, single = _export(module, example_inputs)
    graph = import_exported(ep)
    exe, report = compile_graph(graph, options)
    # weights left unfrozen stay runtime inputs bound to the model's tensors,
    # moved to the GPU once; a model already on the GPU shares its memory
    # (so in-place updates are seen)
    live = dict(module.named_parameters())
    live.update(module.named_buffers())
    params = [(i, live[attrs["param"]].detach().to(exe.device))
              for i, attrs in enumerate(graph.arg_attrs) if "param" in attrs]
    return CompiledModule(exe, report, graph, params, single)
