"""IR, frontend and graph passes (CPU): the producer contracts the HIP backend
consumes, pinned to the reference's test facts (its tests/test_ir.py,
test_freeze.py, test_fusion.py, test_memory_plan.py)."""

import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kiln.api import Options, build_passes
from kiln.frontend.fx_import import Unsupported, import_exported
from kiln.ir import Graph, TensorType, interpret, parse, verify
from kiln.passes.buffers import BufferAssignment, reshape_strides
from kiln.passes.freeze import ConstantFold, FreezeParameters
from kiln.passes.fusion import Fusion
from kiln.passes.manager import PassManager
from kiln.passes.memory_plan import MemoryPlan, align, live_ranges, overlaps
from kiln.passes.partition import OneOpPerKernel
from kiln.passes.simplify import CSE, DCE, Canonicalize
from models.transformer import Block
from test_gpu import random_graph

SRC = """
graph @forward(%arg0: f32[2, 4], %arg1: f32[8, 4] {param = "w"}) -> (f32[2, 8]) {
  %0 = transpose %arg1 {perm = [1, 0]} : f32[4, 8]
  %1 = matmul %arg0, %0 : f32[2, 8]
  %2 = const {value = 0.0} : f32[]
  %3 = maximum %1, %2 : f32[2, 8]
  return %3
}
"""


def imported(model, *xs):
    return import_exported(torch.export.export(model, xs).run_decompositions())


# -- IR --------------------------------------------------------------------------------------

def test_print_parse_roundtrip():
    g = parse(SRC)
    assert str(parse(str(g))) == str(g)


def test_interpret_matches_numpy():
    g = parse(SRC)
    x = np.random.randn(2, 4).astype(np.float32)
    (out,) = interpret(g, x)
    np.testing.assert_allclose(out, np.maximum(x @ g.constants["w"].T, 0), rtol=1e-6)


def test_builder_infers_types():
    g = Graph()
    x = g.add_arg(TensorType((3, 1)), "x")
    y = g.add_arg(TensorType((1, 5)), "y")
    s = g.add_node("add", [x, y])
    r = g.add_node("reduce_sum", [s], {"dims": [1]})
    g.results = [r]
    verify(g)
    assert s.shape == (3, 5) and r.shape == (3, 1)


def test_verifier_rejects_wrong_type():
    with pytest.raises(ValueError, match="does not match"):
        parse(SRC.replace("%1 = matmul %arg0, %0 : f32[2, 8]", "%1 = matmul %arg0, %0 : f32[2, 9]"))


def test_parser_reports_undefined_values():
    with pytest.raises(ValueError, match="undefined"):
        parse(SRC.replace("%3 = maximum %1, %2", "%3 = maximum %9, %2"))


def test_fake_constant_data_is_seeded_by_name():
    a, b = parse(SRC), parse(SRC)
    np.testing.assert_array_equal(a.constants["w"], b.constants["w"])
    assert a.constants["w"].dtype == np.float32 and abs(a.constants["w"].std() - 0.1) < 0.05


def test_reshape_strides_follow_pytorch_views():
    cases = [((8, 16), (48, 1), (8, 2, 8)), ((4, 6), (1, 4), (24,)), ((2, 3, 4), (12, 4, 1), (6, 4)),
             ((2, 1, 3), (3, 3, 1), (1, 2, 3)), ((3, 4), (4, 1), (2, 6))]
    for shape, strides, new in cases:
        base = torch.empty(1000)
        t = torch.as_strided(base, shape, strides)
        try:
            expect = tuple(t.view(new).stride())
        except RuntimeError:
            expect = None
        assert reshape_strides(shape, strides, new) == expect, (shape, strides, new)


def test_importer_rejects_unsupported_ops():
    with pytest.raises(Unsupported):
        imported(torch.nn.Module.__new__(type("M", (torch.nn.Module,), {
            "forward": lambda self, x: torch.cumsum(x, 0)})).__class__(), torch.randn(4))


def test_importer_select():
    class M(torch.nn.Module):
        def forward(self, x):
            return x[1] * 2.0

    g = imported(M(), torch.randn(3, 4))
    x = np.random.randn(3, 4).astype(np.float32)
    np.testing.assert_allclose(interpret(g, x)[0], x[1] * 2.0)


# -- freeze ------------------------------------------------------------------------------------

def test_linear_weight_transpose_is_folded():
    model = torch.nn.Linear(16, 32).eval()
    x = torch.randn(4, 16)
    g = imported(model, x)
    assert any(n.op == "transpose" for n in g.nodes)
    PassManager([FreezeParameters(), ConstantFold(), DCE()]).run(g)
    assert not any(n.op == "transpose" for n in g.nodes)
    assert len(g.args) == 1
    np.testing.assert_array_equal(g.constants["weight.transpose"], model.weight.detach().numpy().T)
    with torch.no_grad():
        np.testing.assert_allclose(interpret(g, x.numpy())[0], model(x).numpy(), rtol=1e-5, atol=1e-6)


def test_freezing_the_transformer_block_preserves_semantics():
    model = Block().eval()
    x = torch.randn(16, 64)
    g = imported(model, x)
    pm = PassManager([Canonicalize(), CSE(), FreezeParameters(), ConstantFold(), Canonicalize(), CSE(), DCE()])
    pm.run(g)
    assert pm.stats["freeze"]["frozen"] == 13          # 12 parameters + the mask buffer
    assert pm.stats["const-fold"]["folded"] == 4       # one transpose per Linear
    with torch.no_grad():
        np.testing.assert_allclose(interpret(g, x.numpy())[0], model(x).numpy(), rtol=1e-4, atol=1e-5)


def test_folding_never_grows_constants():
    g = parse("""
    graph @f(%arg0: f32[64, 64]) -> (f32[64, 64]) {
      %0 = const {value = 2.0} : f32[]
      %1 = expand %0 {shape = [64, 64]} : f32[64, 64]
      %2 = mul %arg0, %1 : f32[64, 64]
      return %2
    }""")
    PassManager([ConstantFold()]).run(g)
    assert any(n.op == "expand" for n in g.nodes)


# -- fusion ------------------------------------------------------------------------------------

def kernels_of(src):
    g = parse(src)
    PassManager([Fusion()]).run(g)
    return [(k.kind, [n.op for n in k.nodes]) for k in g.kernels]


def planned_block(fusion=True, T=16, d=64, nh=4):
    model, x = Block(d=d, nh=nh, T=T).eval(), torch.randn(T, d)
    g = imported(model, x)
    pm = PassManager(build_passes(Options(fusion=fusion)))
    pm.run(g)
    return g, pm, model, x


def test_transformer_block_kernels():
    unfused, _, _, _ = planned_block(fusion=False)
    fused, pm, model, x = planned_block(fusion=True)
    assert len(unfused.kernels) == 44
    assert [k.kind for k in fused.kernels] == ["reduction", "matmul", "copy", "matmul", "reduction", "matmul",
                                               "copy", "matmul", "reduction", "matmul", "matmul"]
    assert [n.op for n in fused.kernels[9].nodes] == ["matmul", "add", "gelu"]
    with torch.no_grad():
        np.testing.assert_allclose(interpret(fused, x.numpy())[0], model(x).numpy(), rtol=1e-4, atol=1e-5)


def test_layernorm_and_softmax_are_one_kernel():
    for fn, x in ((torch.nn.LayerNorm(96).eval(), torch.randn(8, 96)),
                  (type("S", (torch.nn.Module,), {"forward": lambda s, x: F.softmax(x, -1)})(), torch.randn(3, 5, 40))):
        g = imported(fn, x)
        PassManager(build_passes(Options())).run(g)
        assert len(g.kernels) == 1 and g.kernels[0].kind == "reduction"


def test_matmul_with_two_users_is_not_epilogue_fused():
    assert kernels_of("""
    graph @f(%arg0: f32[4, 8], %arg1: f32[8, 16]) -> (f32[4, 16], f32[4, 16]) {
      %0 = matmul %arg0, %arg1 : f32[4, 16]
      %1 = relu %0 : f32[4, 16]
      %2 = exp %0 : f32[4, 16]
      return %1, %2
    }""") == [("matmul", ["matmul"]), ("elementwise", ["relu"]), ("elementwise", ["exp"])]


def test_fusion_never_creates_a_cycle_between_kernels():
    assert kernels_of("""
    graph @f(%arg0: f32[6, 10]) -> (f32[6, 10]) {
      %0 = exp %arg0 : f32[6, 10]
      %1 = reduce_sum %0 {dims = [0]} : f32[1, 10]
      %2 = mul %0, %1 : f32[6, 10]
      return %2
    }""") == [("elementwise", ["exp"]), ("reduction", ["reduce_sum"]), ("elementwise", ["mul"])]


def test_views_end_kernels():
    assert kernels_of("""
    graph @f(%arg0: f32[4, 6]) -> (f32[6, 4]) {
      %0 = exp %arg0 : f32[4, 6]
      %1 = transpose %0 {perm = [1, 0]} : f32[6, 4]
      %2 = relu %1 : f32[6, 4]
      return %2
    }""") == [("elementwise", ["exp"]), ("elementwise", ["relu"])]


def test_kernel_never_reads_its_own_result_through_a_view():
    src = """
    graph @f(%arg0: f32[4, 4]) -> (f32[4, 4]) {
      %0 = add %arg0, %arg0 : f32[4, 4]
      %1 = tanh %0 : f32[4, 4]
      %2 = transpose %1 {perm = [1, 0]} : f32[4, 4]
      %3 = relu %0 : f32[4, 4]
      %4 = sub %2, %3 : f32[4, 4]
      return %4
    }"""
    assert kernels_of(src) == [("elementwise", ["add", "tanh", "relu"]), ("elementwise", ["sub"])]


# -- memory plan ---------------------------------------------------------------------------------

def assert_plan_is_safe(graph):
    ranges = live_ranges(graph)
    spans = {v: (v.node.attrs["offset"], v.node.attrs["offset"] + align(v.type.nbytes)) for v in ranges}
    bufs = list(ranges)
    for i, a in enumerate(bufs):
        assert spans[a][0] % 64 == 0
        assert spans[a][1] <= graph.attrs["arena_bytes"]
        for b in bufs[i + 1:]:
            if overlaps(ranges[a], ranges[b]):
                (s0, e0), (s1, e1) = spans[a], spans[b]
                assert e0 <= s1 or e1 <= s0, f"live buffers share memory: {a} and {b}"


def planned(src, reuse=True):
    g = parse(src)
    pm = PassManager([OneOpPerKernel(), BufferAssignment(), MemoryPlan(reuse=reuse)])
    pm.run(g)
    return g, pm.stats["memory-plan"]


@pytest.mark.parametrize("fusion", [False, True], ids=["unfused", "fused"])
def test_transformer_block_plan(fusion):
    g, pm, _, _ = planned_block(fusion)
    stats = pm.stats["memory-plan"]
    assert_plan_is_safe(g)
    assert stats["arena_bytes"] == stats["lower_bound_bytes"]
    assert stats["naive_bytes"] >= 2 * stats["arena_bytes"]


@pytest.mark.parametrize("T", [128, 512])
def test_gpt2_block_arena_is_the_closed_form(T):
    # arena = peak live set at the softmax kernel: qkv + scores + probs
    # = 4 * (2304 T + 24 T^2) bytes (2.625 MiB at T = 128)
    g, pm, _, _ = planned_block(True, T=T, d=768, nh=12)
    assert g.attrs["arena_bytes"] == 4 * (2304 * T + 24 * T * T)


def test_chain_needs_two_buffers():
    g, stats = planned("""
    graph @chain(%arg0: f32[16, 16]) -> (f32[16, 16]) {
      %0 = exp %arg0 : f32[16, 16]
      %1 = relu %0 : f32[16, 16]
      %2 = neg %1 : f32[16, 16]
      %3 = exp %2 : f32[16, 16]
      %4 = relu %3 : f32[16, 16]
      return %4
    }""")
    assert stats["buffers"] == 4 and stats["naive_bytes"] == 4 * 1024
    assert stats["arena_bytes"] == 2 * 1024
    assert_plan_is_safe(g)


def test_reads_through_views_extend_lifetimes():
    g, _ = planned("""
    graph @f(%arg0: f32[8, 8]) -> (f32[8, 8]) {
      %0 = exp %arg0 : f32[8, 8]
      %1 = relu %0 : f32[8, 8]
      %2 = neg %1 : f32[8, 8]
      %3 = transpose %0 {perm = [1, 0]} : f32[8, 8]
      %4 = add %2, %3 : f32[8, 8]
      return %4
    }""")
    assert live_ranges(g)[g.nodes[0].out] == [0, 3]
    assert_plan_is_safe(g)


def test_no_reuse_gives_every_buffer_its_own_slot():
    _, stats = planned("""
    graph @chain(%arg0: f32[16, 16]) -> (f32[16, 16]) {
      %0 = exp %arg0 : f32[16, 16]
      %1 = relu %0 : f32[16, 16]
      %2 = neg %1 : f32[16, 16]
      return %2
    }""", reuse=False)
    assert stats["arena_bytes"] == stats["naive_bytes"] == 2 * 1024


@pytest.mark.parametrize("fusion", [False, True], ids=["unfused", "fused"])
@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5, 37, 45, 59])
def test_random_graphs_keep_their_meaning_through_the_passes(seed, fusion):
    rng = random.Random(seed)
    g = random_graph(rng, n_ops=rng.randint(6, 22))
    x = np.random.default_rng(seed).standard_normal(g.args[0].shape).astype(np.float32) * 0.5
    expected = interpret(g, x)
    pm = PassManager(build_passes(Options(fusion=fusion)))
    pm.run(g)
    assert_plan_is_safe(g)
    for out, ref in zip(interpret(g, x), expected):
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
