"""Parity of the MI355X HIP backend: every result must match the oracle.

The cases mirror the reference's GPU tests (tests/test_gpu.py:52-169 of the
reference) plus the benchmark configurations at full size. Each compiled result
is compared with
  * the float64 oracle (oracle/interp.py on the imported graph, or the C
    oracle for the named configurations): rtol 1e-4, atol 1e-5 for fp32
    (the tolerance the reference's own GPU tests use), and
  * eager PyTorch fp32 (the reference's check), same tolerance.
"""

import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kiln
import oracle
from kiln.api import Options
from kiln.hip import autotune
from models.transformer import Block, Stack, gpt2_init_
from oracle import interp

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def dev():
    return torch.device("cuda")


def as_tuple(x):
    return x if isinstance(x, tuple) else (x,)


def imported(fn, xs):
    from kiln.frontend.fx_import import import_exported

    module = fn if isinstance(fn, torch.nn.Module) else kiln.api._FnModule(fn)
    module.eval()
    with torch.no_grad():
        ep = torch.export.export(module, tuple(xs)).run_decompositions()
    return import_exported(ep)


def check(fn, *xs, rtol=RTOL, atol=ATOL, **flags):
    """Compile for the GPU, compare with the oracle and with eager torch."""
    compiled = kiln.compile(fn, xs, device="cuda", **flags)
    graph = imported(fn, xs)
    ref = interp.run(graph, *[x.detach().cpu().numpy() for x in xs])
    with torch.no_grad():
        eager = as_tuple(fn(*xs))
    actual = as_tuple(compiled(*xs))
    assert len(actual) == len(ref) == len(eager)
    for a, r, e in zip(actual, ref, eager):
        assert a.device.type == "cuda"
        got = a.detach().cpu().numpy().astype(np.float64)
        np.testing.assert_allclose(got, r, rtol=rtol, atol=atol)
        torch.testing.assert_close(a.cpu(), e.cpu(), rtol=rtol, atol=atol)
    return compiled


W = torch.randn(37, 70)
Y = torch.randn(3, 1)
MASK = torch.full((2, 5000), float("-inf")).triu(1)

CASES = {
    "mlp": (torch.nn.Sequential(torch.nn.Linear(24, 40), torch.nn.GELU(approximate="tanh"),
                                torch.nn.Linear(40, 8)).eval(), (torch.randn(5, 24),)),
    "layernorm": (torch.nn.LayerNorm(48).eval(), (torch.randn(7, 48),)),
    "softmax": (lambda x: F.softmax(x, -1), (torch.randn(3, 5, 33),)),
    "column sum": (lambda x: x.sum(0, keepdim=True) * x, (torch.randn(6, 10),)),
    "full reduction": (lambda x: x.sum((0, 1), keepdim=True) * 2.0, (torch.randn(3, 4),)),
    "reduce dims 0, 2": (lambda x: x.sum((0, 2), keepdim=True) + x.amax(0, keepdim=True), (torch.randn(4, 5, 6),)),
    "views": (lambda x: (x.view(4, 3, 5).transpose(0, 1) * 2.0, x.t()), (torch.randn(12, 5),)),
    "bmm, transposed operand": (lambda a, b: torch.bmm(a, b.transpose(1, 2)),
                                (torch.randn(3, 9, 20), torch.randn(3, 17, 20))),
    "decode, M = 1": (lambda a: F.gelu(a @ W, approximate="tanh"), (torch.randn(1, 37),)),
    "odd K": (lambda a, b: a @ b + 1.0, (torch.randn(33, 45), torch.randn(45, 19))),
    "per-row scalar input": (lambda x: x / (x.sum(-1, keepdim=True) ** 2 + 1.0) + Y, (torch.randn(3, 50),)),
    "multi-shape outputs": (lambda x: (x.exp() * 2, (x.exp() + Y[:2]).sum(-1, keepdim=True)), (torch.randn(2, 9),)),
    "unary ops": (lambda x: torch.tanh(x) + torch.sigmoid(x) + torch.erf(x) + F.gelu(x) + torch.relu(-x),
                  (torch.randn(4, 30) * 3,)),
    "transformer block": (Block(d=32, nh=2, T=8).eval(), (torch.randn(8, 32),)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_matches_reference_cases(name):
    fn, xs = CASES[name]
    check(fn, *xs)


@pytest.mark.parametrize("name", list(CASES))
def test_matches_without_graphs(name):
    fn, xs = CASES[name]
    check(fn, *xs, cuda_graphs=False)


@pytest.mark.parametrize("T", [16, 128])
def test_debug_mode_matches_the_plain_plan(T):
    # Options(debug=True) runs the same kernels launch by launch with NaN
    # poison before each arena buffer's first write and canaries between
    # buffers checked after every launch: a correct plan passes the checks
    # and gives bit for bit the result of the plain plan
    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda", debug=True)
    plain = kiln.compile(model, (x,), device="cuda")
    assert c._exe.guards is not None and c._exe.program.arena_buffers
    xd = x.cuda()
    out = c(xd)
    assert torch.equal(out, plain(xd))
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    np.testing.assert_allclose(out.cpu().numpy(), oracle.block(x.numpy(), params, 12), rtol=RTOL, atol=ATOL)
    assert torch.equal(c(xd), out)


EXP_EXTREMES = [[-200.0, -87.0, -10.0, 0.0, 1e-6, 10.0, 80.0, float("-inf")]]


@pytest.mark.parametrize("graphs", [True, False], ids=["graph", "direct"])
def test_exp_extremes(graphs):
    # the reference's known-answer case (tests/test_compile.py:50-52 there):
    # underflow to 0 (-200, -inf), the smallest normal range (-87), 1 + tiny,
    # and 80 near the fp32 overflow edge, at rtol 1e-5 / atol 1e-30 - through
    # the elementwise tape (KH_OP_EXP) and the softmax row kernel, whose
    # exponentials are exp2((v - max) * log2 e): relative error about
    # |v - max| * 1.2e-7, so the row is also checked scaled by 0.1 (shifted
    # arguments down to -28)
    x = torch.tensor(EXP_EXTREMES)
    c = check(torch.exp, x, rtol=1e-5, atol=1e-30, cuda_graphs=graphs)
    assert c.report.lowering["families"] == {"elementwise": 1}
    for fn in (lambda t: F.softmax(t, -1), lambda t: F.softmax(t * 0.1, -1)):
        c = check(fn, x, rtol=1e-5, atol=1e-30, cuda_graphs=graphs)
        assert c.report.lowering["families"] == {"row": 1}
    # the same values in a 4096-wide row (the one-wave fast path holds the
    # row in registers) and fused after an elementwise op
    wide = torch.randn(3, 4096) * 4
    wide[:, :8] = x
    check(lambda t: torch.exp(t - 1.0), wide, rtol=1e-5, atol=1e-30, cuda_graphs=graphs)
    check(lambda t: F.softmax(t * 0.1, -1), wide, rtol=1e-5, atol=1e-30, cuda_graphs=graphs)


@pytest.mark.parametrize("fn", [torch.nn.LayerNorm(10000).eval(), lambda x: F.softmax(x, -1),
                                lambda x: F.softmax(x + MASK, -1)], ids=["layernorm", "softmax", "masked"])
def test_long_rows_are_chunked(fn):
    # Rows longer than a workgroup chunk are processed in passes, recomputing
    # elementwise values from the inputs instead of storing them.
    x = torch.randn(2, 10000 if isinstance(fn, torch.nn.LayerNorm) else 5000)
    c = check(fn, x)
    assert "(chunked)" in open(c.report.lowering["source"]).read()


def test_fusion_and_memory_planning_apply_on_the_gpu():
    model, x = Block(d=32, nh=2, T=8).eval(), torch.randn(8, 32)
    fused = check(model, x)
    unfused = check(model, x, fusion=False, memory_plan=False)
    assert fused.report.lowering["launches"] < unfused.report.lowering["launches"] / 3
    assert fused.report.arena_bytes < unfused.report.arena_bytes / 4


def test_views_are_strided_loads_not_copies():
    fn = lambda x: x.view(4, 3, 5).transpose(0, 1)[:, 1:3, :] * 2.0
    c = check(fn, torch.randn(12, 5))
    assert not any("copy" in k for k in c.report.kernels)


def test_unfrozen_weights_are_shared_with_a_model_on_the_device():
    model = torch.nn.Linear(16, 8).to(dev())
    x = torch.randn(4, 16, device=dev())
    c = kiln.compile(model, (x,), device="cuda", freeze=False)
    with torch.no_grad():
        model.weight.mul_(2.0)
        torch.testing.assert_close(c(x), model(x), rtol=RTOL, atol=ATOL)


def random_graph(rng, n_ops):
    """Random DAG of elementwise ops, transposes and row centring on a square
    tensor (the reference's generator, tests/test_memory_plan.py:114-137)."""
    from kiln.ir import Graph, TensorType

    g = Graph("random")
    size = rng.choice([4, 8, 12])
    values = [g.add_arg(TensorType((size, size)), "x")]
    for _ in range(n_ops):
        a = rng.choice(values[-4:])
        kind = rng.random()
        if kind < 0.15:
            values.append(g.add_node("transpose", [a], {"perm": [1, 0]}))
        elif kind < 0.3:
            mean = g.add_node("mul", [g.add_node("reduce_sum", [a], {"dims": [1]}), g.scalar(1 / size)])
            values.append(g.add_node("sub", [a, mean]))
        elif kind < 0.6:
            b = rng.choice(values)
            values.append(g.add_node(rng.choice(["add", "sub", "mul", "maximum"]), [a, b]))
        else:
            values.append(g.add_node(rng.choice(["tanh", "sigmoid", "relu", "neg"]), [a]))
    g.results = [values[-1], rng.choice(values[1:-1])]
    return g


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5, 37, 45, 59])
@pytest.mark.parametrize("fusion", [False, True], ids=["unfused", "fused"])
def test_random_graphs(seed, fusion):
    rng = random.Random(seed)
    g = random_graph(rng, n_ops=rng.randint(6, 22))
    x = np.random.default_rng(seed).standard_normal(g.args[0].shape).astype(np.float32) * 0.5
    expected = interp.run(g, x)
    exe, _ = kiln.compile_graph(g, Options(fusion=fusion, device="cuda"))
    for out, ref in zip(exe(torch.from_numpy(x)), expected):
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dim, shape, nan_at", [(-1, (4, 200), (1, 37)), (-1, (3, 5000), (2, 4099)),
                                                 (0, (3000, 5), (1234, 3)), (0, (7, 6), (5, 2))],
                         ids=["row", "chunked row", "column, workgroup tree", "column, per thread"])
def test_max_reductions_propagate_nan(dim, shape, nan_at):
    # One NaN held by a lane other than 0 must reach the result through every
    # cross-lane step (the row kernel's RMAX and both reduce kernels), as in
    # the oracle (np.max) and eager torch.amax.
    x = torch.randn(*shape)
    x[nan_at] = float("nan")
    fn = lambda t: t.amax(dim, keepdim=True) + 0.0 * t
    graph = imported(fn, (x,))
    (ref,) = interp.run(graph, x.numpy())
    out = kiln.compile(fn, (x,), device="cuda")(x).cpu()
    np.testing.assert_allclose(out.numpy(), ref, rtol=RTOL, atol=ATOL, equal_nan=True)
    torch.testing.assert_close(out, fn(x), rtol=RTOL, atol=ATOL, equal_nan=True)
    assert torch.isnan(out).sum() == (shape[1] if dim == -1 else shape[0])


def test_autotune_is_correct_and_cached(monkeypatch):
    from kiln.hip.autotune import GPUAutotuner

    # a shape the shipped table does not hold, so the first compile measures
    model = torch.nn.Sequential(torch.nn.Linear(48, 64), torch.nn.GELU(approximate="tanh")).eval()
    x = torch.randn(20, 48)
    first = check(model, x, autotune=True)
    (entry,) = first.report.autotune
    assert entry["source"] == "tuned" and entry["candidates"] >= 1
    monkeypatch.setattr(GPUAutotuner, "tune", lambda *a, **k: pytest.fail("cached shape re-tuned"))
    second = check(model, x, autotune=True)
    assert second.report.autotune[0]["source"] == "cache"


def test_shipped_table_is_used_before_measuring(monkeypatch):
    from kiln.hip.autotune import GPUAutotuner, shipped_configs

    if not shipped_configs():
        pytest.skip("no shipped tuning table in this tree")
    monkeypatch.setattr(GPUAutotuner, "tune", lambda *a, **k: pytest.fail("shipped shape re-tuned"))
    lin = gpt2_init_(torch.nn.Linear(768, 3072), seed=1).eval()
    x = torch.randn(128, 768)
    c = check(lin, x, autotune=True)
    assert c.report.autotune[0]["source"] == "shipped"


def test_graph_replays_with_new_inputs():
    model = Block(d=64, nh=4, T=16).eval()
    c = kiln.compile(model, (torch.randn(16, 64),), device="cuda")
    assert c.report.lowering["cuda_graphs"]
    for _ in range(3):
        x = torch.randn(16, 64)
        with torch.no_grad():
            torch.testing.assert_close(c(x).cpu(), model(x), rtol=RTOL, atol=ATOL)
    # calls take graph replay or direct launches, whichever measured faster at
    # the first call; both run the same kernels and give the same bits
    assert c._exe.mode in ("graph", "direct")
    x = torch.randn(16, 64)
    outs = {}
    for mode in ("graph", "direct", "graph"):
        c._exe.mode = mode
        outs.setdefault(mode, []).append(c(x))
    assert torch.equal(outs["graph"][0], outs["direct"][0]) and torch.equal(outs["graph"][0], outs["graph"][1])


def test_stored_plan_is_reused_and_bit_identical():
    # the second compile of the same model finds the plan the first one
    # stored (no lowering, no tuning) and computes the same bits
    model = gpt2_init_(Block(256, 4, 64), seed=3).eval()
    x = torch.randn(64, 256)
    first = kiln.compile(model, (x,), device="cuda", autotune=True)
    second = kiln.compile(model, (x,), device="cuda", autotune=True)
    assert first.report.lowering["plan_cache"] == "lowered"
    assert second.report.lowering["plan_cache"] == "stored"
    assert second.report.lowering["source"] == first.report.lowering["source"]
    assert [bytes(l.desc) for l in second._exe.program.launches] == \
        [bytes(l.desc) for l in first._exe.program.launches]
    assert all(e["source"] == "cache" for e in second.report.autotune)
    assert torch.equal(first(x), second(x))
    fresh = kiln.compile(model, (x,), device="cuda", autotune=True, plan_cache=False)
    assert fresh.report.lowering["plan_cache"] == "lowered" and torch.equal(fresh(x), first(x))


def test_native_launch_timing():
    # kh_plan_time: per-launch and whole-plan GPU time from hipGraph replays
    model = gpt2_init_(Block(256, 4, 64), seed=3).eval()
    x = torch.randn(64, 256)
    c = kiln.compile(model, (x,), device="cuda")
    rows = c.profile(x)
    assert [r[0] for r in rows] == c._exe.kernel_names and all(0 < r[3] < 1.0 for r in rows)
    exe = c._exe
    ins = exe._prepare((x,))
    outs = [torch.empty(s, device="cuda") for s in exe.output_shapes]
    from kiln.hip.runtime import current_stream_handle

    total = exe.plan.time([t.data_ptr() for t in ins], [t.data_ptr() for t in outs], current_stream_handle())
    assert 0 < total < 1e-3
    with torch.no_grad():
        torch.testing.assert_close(outs[0].cpu(), model(x), rtol=RTOL, atol=ATOL)


def test_split_k_is_deterministic():
    # split-K partials are summed in split order by whichever workgroup
    # finishes last: repeated runs must be bit-identical.
    a, b = torch.randn(128, 3072, device=dev()), torch.randn(3072, 768, device=dev())
    c = kiln.compile(lambda a, b: a @ b, (a, b), device="cuda", cuda_graphs=False,
                     gpu_matmul_config=lambda *_: {"tile": 2, "splitk": 6})
    first = c(a, b)
    for _ in range(5):
        assert torch.equal(c(a, b), first)
    np.testing.assert_allclose(first.cpu().numpy(), oracle.matmul(a.cpu().numpy(), b.cpu().numpy()),
                               rtol=RTOL, atol=ATOL * 10)


@pytest.mark.parametrize("tile", sorted(autotune.TILES))
def test_every_gemm_tile_configuration(tile):
    # ragged sizes (no dimension a multiple of any tile), then a size with
    # interior tiles (aligned fast path) and ragged edges; bias + residual epilogue
    fn = lambda x, wt, b, r: x @ wt + b + r
    for M, N, K in ((77, 133, 61), (300, 452, 96)):
        x, wt = torch.randn(M, K), torch.randn(K, N) * 0.1
        b, r = torch.randn(N), torch.randn(M, N)
        for splitk in (1, 2):
            c = kiln.compile(fn, (x, wt, b, r), device="cuda", gpu_matmul_config=lambda *_: {"tile": tile,
                                                                                              "splitk": splitk})
            out = c(x, wt, b, r).cpu().numpy()
            ref = oracle.linear(x.numpy(), wt.numpy(), b.numpy(), r.numpy())
            np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("tile", sorted(autotune.SKINNY))
def test_every_skinny_gemm_configuration(tile):
    # skinny-M direct-load kernel: ragged M / N, K a multiple of 4 but not of
    # 16 or of the waves' share, batched constant weights, bias + residual and
    # GELU epilogues; repeated launches agree bit for bit (the waves' partial
    # tiles are summed in a fixed order)
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    for m, n, k in ((21, 40, 68), (128, 768, 768), (77, 133, 1000)):
        torch.manual_seed(m + n + k)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
        x, r = torch.randn(m, k), torch.randn(m, n)
        fn = lambda t, res: lin(t) + res
        c = kiln.compile(fn, (x, r), device="cuda", cuda_graphs=False, gpu_matmul_config=cfg)
        assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
        out = c(x, r)
        ref = oracle.linear(x.numpy(), lin.weight.detach().numpy().T, lin.bias.detach().numpy(), r.numpy())
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=RTOL, atol=ATOL)
        for _ in range(3):
            assert torch.equal(c(x, r), out)
    model = _BatchedConstant(3, 96, 50).eval()
    x = torch.randn(3, 24, 96)
    c = check(model, x, gpu_matmul_config=cfg)
    assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.K_CONTIGUOUS | autotune.SMALL_M)
                                  if autotune.PRECISION[t] == "fp32"])
def test_every_k_contiguous_gemm_configuration(tile):
    # K-contiguous pipelines reading B as a [N][K] copy (the persistent
    # one-workgroup-per-CU kernel and the small-M kernel whose waves split K):
    # ragged M / N (rows and columns past the edge clamped), K a multiple of
    # 32 from one step (fewer steps than waves) to many steps per wave; direct
    # epilogues (bias + residual, bias + GELU) and the tape epilogue (a
    # scale); batched constant weights; repeated launches agree bit for bit
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    for m, n, k in ((21, 40, 32), (77, 133, 96), (300, 452, 160), (256, 768, 768), (128, 200, 3072)):
        torch.manual_seed(m + n + k)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
        x, r = torch.randn(m, k), torch.randn(m, n)
        wt, b = lin.weight.detach().numpy().T, lin.bias.detach().numpy()
        cases = ((lambda t, res: lin(t) + res, (x, r), oracle.linear(x.numpy(), wt, b, r.numpy())),
                 (lambda t: torch.nn.functional.gelu(lin(t), approximate="tanh"), (x,),
                  oracle.linear(x.numpy(), wt, b, act="tanh")),
                 (lambda t, res: lin(t) * 0.5 - res, (x, r), oracle.linear(x.numpy(), wt, b) * 0.5 - r.numpy()))
        for fn, args, ref in cases:
            c = kiln.compile(fn, args, device="cuda", cuda_graphs=False, gpu_matmul_config=cfg)
            assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
            out = c(*args)
            np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=RTOL, atol=ATOL)
            for _ in range(2):
                assert torch.equal(c(*args), out)
    model = _BatchedConstant(3, 96, 50).eval()
    x = torch.randn(3, 24, 96)
    c = check(model, x, gpu_matmul_config=cfg)
    assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary


@pytest.mark.parametrize("variant", range(6))
def test_gemv_variants_and_ragged_sizes(variant):
    # M = 1: every column-block width (0 = chosen from the shape), with and
    # without a K split (two kernels, partials summed in split order); N not
    # a multiple of 4 or of the block, K not a multiple of the k-lanes.
    # Repeated launches (eager and graph replays) must agree bit for bit.
    fn = lambda x, wt, b: x @ wt + b
    for n, k in ((3072, 768), (133, 61), (1030, 999)):
        x, wt, b = torch.randn(1, k), torch.randn(k, n) * 0.1, torch.randn(n)
        ref = oracle.linear(x.numpy(), wt.numpy(), b.numpy())
        for splitk, graphs in ((0, False), (3, False), (3, True)):
            c = kiln.compile(fn, (x, wt, b), device="cuda", cuda_graphs=graphs,
                             gpu_matmul_config=lambda *_: {"tile": variant, "splitk": splitk})
            assert [l.family for l in c._exe.program.launches] == [4]
            first = c(x, wt, b)
            np.testing.assert_allclose(first.cpu().numpy(), ref, rtol=RTOL, atol=ATOL)
            for _ in range(3):
                assert torch.equal(c(x, wt, b), first)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.SMALL_M) if autotune.PRECISION[t] == "fp32"
                                  and autotune.TILES[t][0] <= 4 * autotune.TILES[t][5]])
def test_layernorm_prologue_on_every_small_m_configuration(tile):
    # LayerNorm -> Linear (+ residual) on a small-M configuration: the GEMM
    # takes the row statistics from the A fragments it streams and applies the
    # LayerNorm algebraically (gamma folded into the weight copy, its column
    # sums and beta . W as column constants); the LayerNorm has no launch of
    # its own. Ragged M / N, K from one step to the longest prologue row
    # (1024), with and without affine parameters, rows with mean 3 and with
    # mean 100 (std 1), and rows whose first value is an outlier (20 or 200
    # over N(0, 1) values: a shift by the row's first value would sit 3-27
    # standard deviations from the mean and cost the fp32 sums up to
    # log2(27) bits); repeated launches agree bit for bit
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    for m, n, k, affine, loc, sd, first in ((77, 133, 32, True, 3.0, 2.0, None),
                                            (250, 452, 256, False, 3.0, 2.0, None),
                                            (128, 200, 768, True, 3.0, 2.0, None),
                                            (40, 64, 1024, True, 3.0, 2.0, None),
                                            (64, 96, 768, True, 100.0, 1.0, None),
                                            (64, 768, 768, True, 0.0, 1.0, 20.0),
                                            (64, 768, 768, True, 0.0, 1.0, 200.0),
                                            (50, 96, 256, False, 0.0, 1.0, -200.0)):
        torch.manual_seed(m + k)
        ln = torch.nn.LayerNorm(k, elementwise_affine=affine)
        if affine:
            with torch.no_grad():
                ln.weight.copy_(1.0 + 0.1 * torch.randn(k))
                ln.bias.copy_(0.1 * torch.randn(k))
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
        model = torch.nn.Sequential(ln, lin).eval()
        fn = lambda t, res: model(t) + res
        x, r = loc + sd * torch.randn(m, k), torch.randn(m, n)
        if first is not None:
            x[:, 0] = first
        c = kiln.compile(fn, (x, r), device="cuda", cuda_graphs=False, gpu_matmul_config=cfg)
        summaries = [l.summary for l in c._exe.program.launches]
        assert len(summaries) == 1 and f"tile {tile} " in summaries[0] and "prologue: layernorm" in summaries[0]
        g = ln.weight.detach().numpy() if affine else None
        bt = ln.bias.detach().numpy() if affine else None
        ref = oracle.linear(oracle.layernorm(x.numpy(), g, bt), lin.weight.detach().numpy().T,
                            lin.bias.detach().numpy(), r.numpy())
        out = c(x, r)
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=RTOL, atol=ATOL)
        assert torch.equal(c(x, r), out)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.SMALL_M) if autotune.PRECISION[t] == "fp32"
                                  and autotune.TILES[t][0] <= 4 * autotune.TILES[t][5]])
def test_layernorm_prologue_non_finite_rows(tile):
    # A row holding NaN, +inf, -inf or both infinities normalises to NaN in
    # every element (the oracle's LayerNorm: its mean or variance is not
    # finite), so its product row is NaN in every column, whichever element
    # is not finite - also the row's first value, the shift the folded
    # LayerNorm subtracts. The row statistics are merged per row across lanes
    # and waves, so the other rows of the same tiles stay exact
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    m, n, k = 70, 90, 256
    torch.manual_seed(11)
    ln = torch.nn.LayerNorm(k)
    with torch.no_grad():
        ln.weight.copy_(1.0 + 0.1 * torch.randn(k))
        ln.bias.copy_(0.1 * torch.randn(k))
    lin = gpt2_init_(torch.nn.Linear(k, n), seed=5).eval()
    model = torch.nn.Sequential(ln, lin).eval()
    x = 3.0 + 2.0 * torch.randn(m, k)
    bad = {5: [(17, math.nan)], 20: [(0, math.inf)], 33: [(200, -math.inf)], 40: [(3, math.inf), (90, -math.inf)],
           47: [(0, math.nan)], 69: [(255, math.nan)]}
    for row, cells in bad.items():
        for col, v in cells:
            x[row, col] = v
    c = kiln.compile(model, (x,), device="cuda", cuda_graphs=False, gpu_matmul_config=cfg)
    summaries = [l.summary for l in c._exe.program.launches]
    assert len(summaries) == 1 and f"tile {tile} " in summaries[0] and "prologue: layernorm" in summaries[0]
    ref = oracle.linear(oracle.layernorm(x.numpy(), ln.weight.detach().numpy(), ln.bias.detach().numpy()),
                        lin.weight.detach().numpy().T, lin.bias.detach().numpy())
    assert np.isnan(ref[sorted(bad)]).all() and np.isfinite(np.delete(ref, sorted(bad), axis=0)).all()
    out = c(x).cpu().numpy()
    np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL, equal_nan=True)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.SMALL_M) if autotune.PRECISION[t] == "fp32"
                                  and autotune.TILES[t][0] <= 4 * autotune.TILES[t][5]])
def test_layernorm_prologue_through_a_row_reshape(tile):
    # LayerNorm over [B, T, K] feeding a Linear (A = its output reshaped to
    # [B*T, K]): the product reads the LayerNorm's input with the merged row
    # stride and runs the LayerNorm as its prologue
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    torch.manual_seed(tile)
    ln = torch.nn.LayerNorm(256)
    with torch.no_grad():
        ln.weight.copy_(1.0 + 0.1 * torch.randn(256))
        ln.bias.copy_(0.1 * torch.randn(256))
    lin = gpt2_init_(torch.nn.Linear(256, 120), seed=2).eval()
    model = torch.nn.Sequential(ln, lin).eval()
    x = 3.0 + 2.0 * torch.randn(3, 45, 256)
    c = kiln.compile(model, (x,), device="cuda", cuda_graphs=False, gpu_matmul_config=cfg)
    summaries = [l.summary for l in c._exe.program.launches]
    assert f"tile {tile} " in summaries[0] and "prologue: layernorm" in summaries[0]
    assert not any("layernorm rows" in s for s in summaries)
    ref = oracle.linear(oracle.layernorm(x.reshape(-1, 256).numpy(), ln.weight.detach().numpy(),
                                         ln.bias.detach().numpy()),
                        lin.weight.detach().numpy().T, lin.bias.detach().numpy()).reshape(3, 45, 120)
    np.testing.assert_allclose(c(x).cpu().numpy(), ref, rtol=RTOL, atol=ATOL)


class _BatchedConstant(torch.nn.Module):
    def __init__(self, batch, k, n):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(batch, k, n) * 0.1)

    def forward(self, x):
        return torch.matmul(x, self.w) * 0.5


@pytest.mark.parametrize("k, n, batch", [(768, 2304, 1), (3072, 768, 1), (9000, 70, 1), (64, 130, 3), (12, 5, 1)])
def test_k_contiguous_gemv(k, n, batch):
    # M = 1 with a constant weight: the weight is read as a [batch][N][K] copy
    # by the K-contiguous kernel (one pass of R float4 per lane; several
    # passes beyond K = 8192; N not a multiple of 4; batched constants);
    # eager and graph-replayed launches agree bit for bit
    torch.manual_seed(k + n)
    if batch == 1:
        model = torch.nn.Sequential(torch.nn.Linear(k, n), torch.nn.GELU(approximate="tanh")).eval()
        x = torch.randn(1, k)
    else:
        model = _BatchedConstant(batch, k, n).eval()
        x = torch.randn(batch, 1, k)
    c = check(model, x)
    assert c.report.lowering["families"] == {"gemv": 1}
    assert any("@nk:" in name for name in c._exe.program.derived)
    first = c(x)
    for graphs in (False, True):
        c2 = kiln.compile(model, (x,), device="cuda", cuda_graphs=graphs)
        for _ in range(3):
            assert torch.equal(c2(x), first)


def test_batched_gemv_with_strided_weights():
    # batch 3, M = 1, B read through a transposed view (no 128-bit column quads)
    check(lambda a, b: torch.bmm(a, b.transpose(1, 2)) * 0.5, torch.randn(3, 1, 300), torch.randn(3, 70, 300))


def test_strided_and_broadcast_gemm_operands():
    # A transposed (k-stride != 1), B a column slice, bias broadcast over rows
    a, b = torch.randn(40, 30), torch.randn(50, 70)
    fn = lambda a, b: a.t() @ b[:40, 3:64] + b[0, 3:64]
    check(fn, a, b)


# -- benchmark configurations at full size -----------------------------------------------

def test_config_linear_bias_gelu():
    torch.manual_seed(0)
    lin = torch.nn.Linear(768, 3072)
    gpt2_init_(lin, seed=0)
    model = torch.nn.Sequential(lin, torch.nn.GELU()).eval()
    x = torch.randn(128, 768)
    c = kiln.compile(model, (x,), device="cuda")
    out = c(x).cpu().numpy()
    ref = oracle.linear(x.numpy(), lin.weight.detach().numpy().T, lin.bias.detach().numpy(), act="erf")
    np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)


def test_config_fused_memory_bound_ops():
    torch.manual_seed(0)
    x, b = torch.randn(2048, 3072), torch.randn(3072)
    c = kiln.compile(lambda t: F.gelu(t + b, approximate="tanh"), (x,), device="cuda")
    np.testing.assert_allclose(c(x).cpu().numpy(), oracle.bias_gelu(x.numpy(), b.numpy()), rtol=RTOL, atol=ATOL)

    ln = torch.nn.LayerNorm(768).eval()
    with torch.no_grad():
        ln.weight.copy_(1 + torch.randn(768) * 0.02)
        ln.bias.copy_(torch.randn(768) * 0.02)
    x = torch.randn(2048, 768)
    c = kiln.compile(ln, (x,), device="cuda")
    assert "layernorm" in open(c.report.lowering["source"]).read()
    ref = oracle.layernorm(x.numpy(), ln.weight.detach().numpy(), ln.bias.detach().numpy())
    np.testing.assert_allclose(c(x).cpu().numpy(), ref, rtol=RTOL, atol=ATOL)

    x = torch.randn(12, 512, 512)
    c = kiln.compile(lambda t: F.softmax(t * 0.125, -1), (x,), device="cuda")
    assert "softmax" in open(c.report.lowering["source"]).read()
    np.testing.assert_allclose(c(x).cpu().numpy(), oracle.softmax(x.numpy(), 0.125), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("mnk", [(2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768),
                                 (128, 768, 3072), (1, 3072, 768)])
def test_config_gemm_sweep(mnk):
    m, n, k = mnk
    torch.manual_seed(0)
    lin = torch.nn.Linear(k, n)
    gpt2_init_(lin, seed=1)
    lin.eval()
    x = torch.randn(m, k)
    c = kiln.compile(lin, (x,), device="cuda")
    ref = oracle.linear(x.numpy(), lin.weight.detach().numpy().T, lin.bias.detach().numpy())
    np.testing.assert_allclose(c(x).cpu().numpy(), ref, rtol=RTOL, atol=ATOL)


def _block(T, seed=0):
    torch.manual_seed(seed)
    return gpt2_init_(Block(768, 12, T), seed=seed).eval()


@pytest.mark.parametrize("T", [128, 512])
def test_config_gpt2_block(T):
    model = _block(T)
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda")
    # attention fused into one launch; a LayerNorm feeding a small-M GEMM
    # runs as that GEMM's prologue (both at T = 128)
    n_pro = sum("prologue: layernorm" in l.summary for l in c._exe.program.launches)
    assert c.report.lowering["launches"] == 7 - n_pro and (T != 128 or n_pro == 2)
    out = c(x).cpu().numpy()
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    ref = oracle.block(x.numpy(), params, 12)
    np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("T", [1024, 2048])
def test_config_gpt2_block_long(T):
    # the whole [T, 768] output against the C oracle (float64 inside), and
    # against eager PyTorch fp32
    model = _block(T)
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda")
    out = c(x).cpu()
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    ref = oracle.block(x.numpy(), params, 12)
    np.testing.assert_allclose(out.numpy(), ref, rtol=RTOL, atol=ATOL)
    with torch.no_grad():
        torch.testing.assert_close(out, model(x), rtol=RTOL, atol=ATOL)


class _LayerTaps(torch.nn.Module):
    """A Stack that returns every block's output and the final LayerNorm's."""

    def __init__(self, stack):
        super().__init__()
        self.stack = stack

    def forward(self, x):
        outs = []
        for blk in self.stack.blocks:
            x = blk(x)
            outs.append(x)
        outs.append(self.stack.ln_f(x))
        return tuple(outs)


# Per-layer error of the 12-layer stack, as max |y - y64| / max |y64| against
# a float64 run of the same weights and input (torch float64 on the CPU).
# Eager PyTorch fp32 has an error of its own against float64 (fp32 rounding
# compounding through 12 layers); kiln must stay within STACK_ERR_FACTOR of
# eager's error at every layer, and the final output within the per-kernel
# bar (rtol 1e-4, atol 1e-5) of float64, element by element.
STACK_ERR_FACTOR = 2.0
STACK_ERR_FLOOR = 1e-6


@pytest.mark.parametrize("T", [1024, 1], ids=["prefill_1024", "decode_1"])
def test_config_stack_12_layers_against_float64(T):
    import copy

    torch.manual_seed(0)
    model = gpt2_init_(Stack(12, 768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    taps = _LayerTaps(model).eval()
    c = kiln.compile(taps, (x,), device="cuda")
    if T == 1:
        assert any(l.family == 4 for l in c._exe.program.launches)   # the GEMV path
    got = [t.cpu().double() for t in c(x)]
    with torch.no_grad():
        ref = _LayerTaps(copy.deepcopy(model).double()).eval()(x.double())
        eager = [t.cpu().double() for t in copy.deepcopy(taps).cuda()(x.cuda())]
    worst = 0.0
    for layer, (g, r, e) in enumerate(zip(got, ref, eager)):
        scale = float(r.abs().max())
        k_err, e_err = float((g - r).abs().max()) / scale, float((e - r).abs().max()) / scale
        print(f"stack T={T} layer {layer}: kiln {k_err:.2e}, eager fp32 {e_err:.2e} of max |y64|", flush=True)
        assert k_err <= max(STACK_ERR_FACTOR * e_err, STACK_ERR_FLOOR), (layer, k_err, e_err)
        worst = max(worst, k_err / max(e_err, 1e-12))
    np.testing.assert_allclose(got[-1].numpy(), ref[-1].numpy(), rtol=RTOL, atol=ATOL)
    print(f"stack T={T}: worst kiln/eager error ratio {worst:.2f}", flush=True)


@pytest.mark.parametrize("k, n, affine, bias", [(768, 2304, True, True), (61, 37, True, False),
                                               (64, 48, False, True), (3072, 768, True, True)])
def test_layernorm_prologue_of_a_gemv(k, n, affine, bias):
    """LayerNorm -> Linear at one row runs as one GEMV with the LayerNorm as
    its prologue; checked against the oracle interpreter and eager torch."""
    torch.manual_seed(0)
    ln = torch.nn.LayerNorm(k, elementwise_affine=affine)
    if affine:
        with torch.no_grad():
            ln.weight.copy_(1 + 0.1 * torch.randn(k))
            ln.bias.copy_(0.1 * torch.randn(k))
    model = torch.nn.Sequential(ln, torch.nn.Linear(k, n, bias=bias), torch.nn.GELU(approximate="tanh")).eval()
    x = 3.0 + 2.0 * torch.randn(1, k)
    c = check(model, x)
    assert c.report.lowering["launches"] == 1 and c.report.lowering["families"] == {"gemv": 1}


@pytest.mark.parametrize("cells", [[(5, math.nan)], [(0, math.inf)], [(700, -math.inf)], [(3, math.inf), (9, -math.inf)]])
def test_layernorm_prologue_of_a_gemv_non_finite_row(cells):
    # a row holding NaN or infinities normalises to NaN in every element (the
    # oracle's LayerNorm), so every output of the GEMV is NaN
    torch.manual_seed(1)
    k, n = 768, 300
    ln = torch.nn.LayerNorm(k)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(k))
        ln.bias.copy_(0.1 * torch.randn(k))
    lin = torch.nn.Linear(k, n)
    model = torch.nn.Sequential(ln, lin).eval()
    x = 3.0 + 2.0 * torch.randn(1, k)
    for col, v in cells:
        x[0, col] = v
    c = kiln.compile(model, (x,), device="cuda")
    assert c.report.lowering["launches"] == 1 and c.report.lowering["families"] == {"gemv": 1}
    ref = oracle.linear(oracle.layernorm(x.numpy(), ln.weight.detach().numpy(), ln.bias.detach().numpy()),
                        lin.weight.detach().numpy().T, lin.bias.detach().numpy())
    assert np.isnan(ref).all()
    assert torch.isnan(c(x)).all()
