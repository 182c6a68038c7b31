"""torch.compile(backend=kiln.backend) on the CPU side: fallback and strict
mode follow the reference bridge (tests/test_compile.py:108-130 there), and
the graphs aot_autograd hands over import and lower to the HIP families
without a GPU (weights arrive as graph inputs, freezing off)."""

import pytest
import torch
from torch._dynamo.backends.common import aot_autograd

import kiln
from kiln.api import Options, build_passes
from kiln.frontend.fx_import import import_fx
from kiln.hip import lib as kl
from kiln.hip.attention import FuseAttention
from kiln.hip.lowering import lower_graph
from kiln.passes.manager import PassManager
from models.transformer import Block


def test_cpu_inputs_fall_back_to_eager_with_a_warning(monkeypatch):
    monkeypatch.setenv("KILN_STRICT", "0")
    kiln.stats.update(compiled=0, fallback=0)
    torch._dynamo.reset()
    model = torch.nn.Sequential(torch.nn.Linear(8, 16), torch.nn.GELU()).eval()
    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)
    x = torch.randn(4, 8)
    with pytest.warns(UserWarning, match="falling back"):
        with torch.no_grad():
            torch.testing.assert_close(compiled(x), model(x), rtol=1e-4, atol=1e-5)
    assert kiln.stats == {"compiled": 0, "fallback": 1}


def test_unsupported_ops_fall_back(monkeypatch):
    monkeypatch.setenv("KILN_STRICT", "0")
    kiln.stats.update(compiled=0, fallback=0)
    torch._dynamo.reset()
    fn = lambda x: torch.cumsum(x, 0)
    compiled = torch.compile(fn, backend=kiln.backend, dynamic=False)
    x = torch.randn(5)
    with pytest.warns(UserWarning, match="falling back"):
        with torch.no_grad():
            torch.testing.assert_close(compiled(x), fn(x))
    assert kiln.stats["fallback"] == 1


def test_strict_mode_raises(monkeypatch):
    monkeypatch.setenv("KILN_STRICT", "1")
    torch._dynamo.reset()
    compiled = torch.compile(lambda x: x * 2 + 1, backend=kiln.backend, dynamic=False)
    with pytest.raises(Exception, match="GPU only"):
        compiled(torch.randn(3))
    torch._dynamo.reset()


def _forward_graphs(model, x):
    """The forward graphs aot_autograd gives a backend, captured on the CPU."""
    seen = []

    def grab(gm, example_inputs):
        seen.append(gm)
        return gm.forward

    torch._dynamo.reset()
    compiled = torch.compile(model, backend=aot_autograd(fw_compiler=grab), dynamic=False)
    with torch.no_grad():
        compiled(x)
    torch._dynamo.reset()
    return seen


def _lower(gm):
    g = import_fx(gm)
    passes = build_passes(Options(device="cuda", freeze=False))
    passes.insert(len(passes) - 1, FuseAttention())
    PassManager(passes).run(g)
    return lower_graph(g)


def test_linear_gelu_graph_lowers_with_the_weight_as_an_input():
    model = torch.nn.Sequential(torch.nn.Linear(8, 16), torch.nn.GELU()).eval()
    (gm,) = _forward_graphs(model, torch.randn(4, 8))
    # weight and bias are runtime inputs (lifted parameters), not constants
    g = import_fx(gm)
    assert len(g.args) == 3 and not g.constants
    prog = _lower(gm)
    # the weight is read in its [out, in] layout: one transposing copy, then
    # the GEMM with bias and GELU in its epilogue
    assert [kl.FAMILY_NAMES[l.family] for l in prog.launches] == ["elementwise", "gemm"]
    assert "gelu" in prog.launches[1].summary


def test_gpt2_block_graph_lowers_with_fused_attention():
    T = 64
    (gm,) = _forward_graphs(Block(768, 12, T).eval(), torch.randn(T, 768))
    prog = _lower(gm)
    fams = [kl.FAMILY_NAMES[l.family] for l in prog.launches]
    assert fams.count("attention") == 1 and fams.count("gemm") == 4, fams
