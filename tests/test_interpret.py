"""The plan's meaning on the CPU (``KILN_HIP_INTERPRET=1``: the library's
kh_plan_run_host). Every case goes through the real compile path - passes,
lowering, plan validation in the library - and the host interpreter then
executes the descriptors, addressing and tapes element by element; results
are checked against the oracle at the GPU tests' tolerance. This is how the
CPU suite catches a lowering or addressing mistake without a GPU, as the
reference's interpreter switch does for its GPU tests (tests/conftest.py:11-15
there)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kiln
import oracle
from kiln.hip import bf16
from models.transformer import Block, Stack, gpt2_init_
from oracle import interp
from test_gpu import ATOL, CASES, RTOL, as_tuple, imported, random_graph


@pytest.fixture(autouse=True)
def _interpreting(monkeypatch):
    monkeypatch.setenv("KILN_HIP_INTERPRET", "1")
    yield


def check(fn, *xs, rtol=RTOL, atol=ATOL, **flags):
    compiled = kiln.compile(fn, xs, device="cuda", **flags)
    ref = interp.run(imported(fn, xs), *[x.numpy() for x in xs])
    got = as_tuple(compiled(*xs))
    assert len(got) == len(ref)
    for a, r in zip(got, ref):
        assert a.device.type == "cpu"
        np.testing.assert_allclose(a.numpy().astype(np.float64), r, rtol=rtol, atol=atol)
    return compiled


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("fusion", [True, False], ids=["fused", "unfused"])
def test_reference_cases(name, fusion):
    fn, xs = CASES[name]
    check(fn, *xs, fusion=fusion)


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5, 37, 45, 59])
def test_random_graphs(seed):
    import random

    from kiln.api import Options

    rng = random.Random(seed)
    g = random_graph(rng, n_ops=rng.randint(6, 22))
    x = np.random.default_rng(seed).standard_normal(g.args[0].shape).astype(np.float32) * 0.5
    expected = interp.run(g, x)
    exe, _ = kiln.compile_graph(g, Options(device="cuda"))
    for out, ref in zip(exe(torch.from_numpy(x)), expected):
        np.testing.assert_allclose(out.numpy(), ref, rtol=RTOL, atol=ATOL)


def test_long_rows_run_in_chunks():
    # chunked multi-pass rows: the interpreter poisons per-column values
    # between passes, so a pass reading a stale value would show as NaN
    x = torch.randn(2, 5000)
    c = check(lambda t: F.softmax(t, -1), x)
    assert "(chunked)" in open(c.report.lowering["source"]).read()
    check(torch.nn.LayerNorm(6000).eval(), torch.randn(3, 6000))


def test_max_reductions_propagate_nan():
    x = torch.randn(300, 7)
    x[123, 2] = float("nan")
    for dim in (0, -1):
        fn = lambda t: t.amax(dim, keepdim=True) + 0.0 * t
        ref = interp.run(imported(fn, (x,)), x.numpy())[0]
        np.testing.assert_allclose(kiln.compile(fn, (x,), device="cuda")(x).numpy(), ref, equal_nan=True)


@pytest.mark.parametrize("T", [16, 48])
def test_gpt2_block_against_the_c_oracle(T):
    torch.manual_seed(0)
    model = gpt2_init_(Block(128, 4, T), seed=0).eval()
    x = torch.randn(T, 128)
    c = kiln.compile(model, (x,), device="cuda")
    assert c.report.lowering["families"].get("attention") == 1
    # both LayerNorms run inside the small-M GEMMs that read them (folded
    # gamma / beta constants, row statistics in the product)
    src = open(c.report.lowering["source"]).read()
    assert src.count("prologue: layernorm") == 2 and "layernorm rows" not in src
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    np.testing.assert_allclose(c(x).numpy(), oracle.block(x.numpy(), params, 4), rtol=RTOL, atol=ATOL)


def test_decode_stack_runs_gemv_prologues():
    # M = 1: LayerNorm and one-query attention as GEMV prologues, K-contiguous weights
    torch.manual_seed(0)
    model = gpt2_init_(Stack(2, 128, 4, 1), seed=0).eval()
    x = torch.randn(1, 128)
    c = kiln.compile(model, (x,), device="cuda")
    src = open(c.report.lowering["source"]).read()
    assert "prologue: layernorm" in src and "prologue: attention" in src
    h = x.numpy()
    for blk in model.blocks:
        h = oracle.block(h, {k: v.numpy() for k, v in blk.state_dict().items()}, 4)
    sd = model.ln_f.state_dict()
    ref = oracle.layernorm(h, sd["weight"].numpy(), sd["bias"].numpy())
    np.testing.assert_allclose(c(x).numpy(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("shape, perm, fused", [((3, 20, 64), None, True), ((2, 5, 1, 64), None, True),
                                                ((1, 1, 64), None, True), ((20, 3, 64), (1, 0, 2), False)])
def test_layernorm_prologue_through_a_row_reshape(shape, perm, fused):
    # LayerNorm over [B, T, K] feeding a Linear: the product's A is the
    # LayerNorm's output reshaped to [B*T, K]; the product runs the LayerNorm as
    # its prologue and reads x with the merged row stride - unless x's leading
    # dims do not merge into one stride (a permuted input), when the LayerNorm
    # stays a row kernel
    torch.manual_seed(3)
    ln = torch.nn.LayerNorm(64)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(64))
        ln.bias.copy_(0.1 * torch.randn(64))
    lin = torch.nn.Linear(64, 48)
    model = torch.nn.Sequential(ln, lin).eval()
    fn = (lambda t: model(t.permute(*perm))) if perm else model
    x = 3.0 + 2.0 * torch.randn(*shape)
    c = check(fn, x)
    src = open(c.report.lowering["source"]).read()
    assert ("prologue: layernorm" in src) == fused and ("layernorm rows" in src) != fused


def test_exp_extremes():
    # the reference's known-answer case (tests/test_compile.py:50-52 there)
    # through the elementwise tape and the softmax row pass
    x = torch.tensor([[-200.0, -87.0, -10.0, 0.0, 1e-6, 10.0, 80.0, float("-inf")]])
    for fn in (torch.exp, lambda t: F.softmax(t, -1), lambda t: F.softmax(t * 0.1, -1)):
        check(fn, x, rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("first", [20.0, 200.0, -200.0])
def test_layernorm_prologue_rows_with_an_outlier_first_value(first):
    # rows of N(0, 1) values whose first value is an outlier: the folded
    # constants (gamma * W, its column sums, beta . W) stand for the same
    # LayerNorm -> Linear whatever the row's spread
    torch.manual_seed(7)
    ln = torch.nn.LayerNorm(256)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(256))
        ln.bias.copy_(0.1 * torch.randn(256))
    lin = gpt2_init_(torch.nn.Linear(256, 96), seed=1)
    model = torch.nn.Sequential(ln, lin).eval()
    x = torch.randn(40, 256)
    x[:, 0] = first
    c = check(model, x)
    assert "prologue: layernorm" in open(c.report.lowering["source"]).read()


@pytest.mark.parametrize("precision", ["bf16", "bf16x3"])
def test_bf16_products_round_as_the_mfma_variants(precision):
    torch.manual_seed(0)
    lin = gpt2_init_(torch.nn.Linear(96, 40), seed=2).eval()
    x = torch.randn(24, 96)
    c = kiln.compile(lin, (x,), device="cuda", matmul_precision=precision)
    w = lin.weight.detach().numpy().T
    if precision == "bf16":
        # against the product of the bf16-rounded inputs, in float64
        xr, wr = bf16.bf16_value(bf16.bf16_bits(x.numpy())), bf16.bf16_value(bf16.bf16_bits(w))
        ref = xr.astype(np.float64) @ wr.astype(np.float64) + lin.bias.detach().numpy()
        np.testing.assert_allclose(c(x).numpy(), ref, rtol=1e-5, atol=1e-6)
    else:
        ref = oracle.linear(x.numpy(), w, lin.bias.detach().numpy())
        np.testing.assert_allclose(c(x).numpy(), ref, rtol=RTOL, atol=ATOL)


def test_interpreter_is_never_a_gpu_path():
    from kiln.hip.interpret import refuse

    with pytest.raises(RuntimeError, match="KILN_HIP_INTERPRET"):
        refuse("bench.py")


@pytest.mark.parametrize("tile", [15, 34, 26])
def test_other_precision_config_on_two_activations(tile):
    # a configuration of another precision (bf16 / bf16x3 tiles asked for an
    # fp32 product) falls back to the fp32 default; with two activations that
    # default must not be a configuration reading B as a [N][K] constant copy
    from kiln.hip import autotune

    for m in (77, 128, 300):
        a, b = torch.randn(m, 96), torch.randn(96, 130)
        c = check(lambda x, y: x @ y, a, b, gpu_matmul_config=lambda *_: {"tile": tile, "splitk": 1})
        (launch,) = c._exe.program.launches
        chosen = int(launch.summary.split(" tile ")[1].split()[0])
        assert chosen not in autotune.NK_B and autotune.PRECISION[chosen] == "fp32"


@pytest.mark.parametrize("tile", [47, 49, 53])
def test_skinny_gemm_lowering(tile):
    # skinny-M configurations read the weight as a [N][K] copy; a product of
    # two activations cannot use them and keeps a tiled configuration
    lin = gpt2_init_(torch.nn.Linear(68, 40), seed=1).eval()
    x = torch.randn(21, 68)
    model = torch.nn.Sequential(lin, torch.nn.GELU(approximate="tanh")).eval()
    c = check(model, x, gpu_matmul_config=lambda *_: {"tile": tile, "splitk": 3})
    (launch,) = c._exe.program.launches
    assert f"tile {tile} splitk" in launch.summary and any("@nk:" in n for n in c._exe.program.derived)
    c2 = check(lambda a, b: a @ b, torch.randn(21, 68), torch.randn(68, 40),
               gpu_matmul_config=lambda *_: {"tile": tile, "splitk": 1})
    assert f"tile {tile} " not in c2._exe.program.launches[0].summary


def test_decode_stack_forms_one_gemv_chain():
    # every GEMV of the decode stack reads the whole output of the one before
    # (x, or q / k / v of the attention prologue), so the library chains all of
    # them; the final LayerNorm is a row launch after the chain. On the host
    # the chain is not bound (no GPU) and the launches run one by one.
    torch.manual_seed(0)
    model = gpt2_init_(Stack(3, 128, 4, 1), seed=0).eval()
    x = torch.randn(1, 128)
    c = kiln.compile(model, (x,), device="cuda", gemv_chains=True)
    low = c.report.lowering
    assert low["launches"] == 13
    assert low["gemv_chains"] == [(0, 12)]
    off = kiln.compile(model, (x,), device="cuda")   # chains are opt-in
    assert off.report.lowering["gemv_chains"] == []
    np.testing.assert_array_equal(c(x).numpy(), off(x).numpy())


def test_gemv_chain_needs_the_whole_previous_output():
    # the second product reads half of the first one's output: not chained
    # (a stage's waves must have waited for every output of the stage before)
    w1 = torch.randn(64, 96) * 0.1
    w2 = torch.randn(16, 32) * 0.1
    w3 = torch.randn(16, 64) * 0.1

    def half(x):
        y = F.linear(x, w1)
        return F.linear(y[:, :32], w2)

    def whole(x):
        return F.linear(F.linear(x, w1), w3)

    x = torch.randn(1, 96)
    assert check(half, x, gemv_chains=True).report.lowering["gemv_chains"] == []
    assert check(whole, x, gemv_chains=True).report.lowering["gemv_chains"] == [(0, 2)]


def test_debug_mode_runs_launch_by_launch_against_the_oracle():
    # Options(debug=True): guards between arena buffers, NaN poison before
    # each buffer's first write, canaries checked after every launch; a
    # correct plan passes them and gives the oracle's result
    torch.manual_seed(0)
    model = gpt2_init_(Block(128, 4, 16), seed=0).eval()
    x = torch.randn(16, 128)
    c = kiln.compile(model, (x,), device="cuda", debug=True)
    plain = kiln.compile(model, (x,), device="cuda")
    assert c.report.arena_bytes > plain.report.arena_bytes   # the guards take room
    assert c._exe.program.arena_buffers
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    np.testing.assert_allclose(c(x).numpy(), oracle.block(x.numpy(), params, 4), rtol=RTOL, atol=ATOL)


def _debug_exe(program, c):
    from kiln.hip.interpret import HostExecutable

    exe = c._exe
    return HostExecutable(program, c.report.arena_bytes, c.graph.constants, exe.input_shapes, exe.output_shapes,
                          debug=True)


def test_debug_mode_catches_a_write_past_a_buffer():
    # plant a mistake in the plan (CPU): the first launch's store moved 8
    # floats along the arena, so it writes into the next guard bytes
    import copy

    from kiln.hip import lib as kl

    fn = lambda t: torch.exp(t * 2.0) + 1.0
    x = torch.randn(4, 64)
    c = kiln.compile(fn, (x,), device="cuda", fusion=False, debug=True)
    np.testing.assert_allclose(c(x).numpy(), fn(x).numpy(), rtol=RTOL, atol=ATOL)
    program = copy.deepcopy(c._exe.program)
    d = program.launches[0].desc
    store = [j for j in range(d.n_refs) if d.refs[j].base == kl.BASE_ARENA]
    assert len(store) == 1
    d.refs[store[0]].offset += 8
    with pytest.raises(RuntimeError, match="wrote past the end of arena buffer"):
        _debug_exe(program, c)(x)


def test_debug_mode_poisons_a_buffer_read_before_it_is_written():
    # plant a mistake in the plan (CPU): the second launch reads its input 8
    # floats early, from bytes no launch of this call has written (the guard
    # and the previous buffer's tail): NaN reaches the output
    import copy

    from kiln.hip import lib as kl

    fn = lambda t: torch.exp(t * 2.0) + 1.0
    x = torch.randn(4, 64)
    c = kiln.compile(fn, (x,), device="cuda", fusion=False, debug=True)
    program = copy.deepcopy(c._exe.program)
    d = program.launches[1].desc
    load = [j for j in range(d.n_refs) if d.refs[j].base == kl.BASE_ARENA]
    d.refs[load[0]].offset += 64            # one row further (elements): the last row reads the guard
    out = _debug_exe(program, c)(x)[0].numpy()
    assert np.isnan(out[-1]).all() and np.isfinite(out[:-1]).all()


def _no_bf16_storage(monkeypatch):
    from kiln.hip import lowering

    monkeypatch.setattr(lowering._Lowerer, "plan_bf16_storage", lambda self: set())


def test_bf16_storage_between_producers_and_products_gives_the_same_bits(monkeypatch):
    # bf16 plans on the 64-deep product configurations: the LayerNorms, the
    # attention and the MLP-up product round their outputs to bf16 when a
    # bf16 product is their only reader, and the QKV product rounds q, k, v
    # for the attention's bf16 products; the readers take them as bf16. The
    # rounding is the one the readers would do when they form their operands,
    # so the result is bit for bit the one of the same plan with fp32 storage
    torch.manual_seed(0)
    model = gpt2_init_(Block(128, 4, 16), seed=0).eval()
    x = torch.randn(16, 128)
    cfg = lambda *_: {"tile": 99, "splitk": 1}
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    summaries = [l.summary for l in c._exe.program.launches]
    assert sum("A:bf16" in s for s in summaries) == 4, summaries
    assert sum("out:bf16" in s for s in summaries) == 5, summaries   # 2 LayerNorms, QKV, attention, MLP up
    assert any("heads" in s and "qkv:bf16" in s for s in summaries), summaries
    got = c(x)
    _no_bf16_storage(monkeypatch)
    plain = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    assert not any("bf16" in s.split("bf16", 1)[-1] for s in [l.summary for l in plain._exe.program.launches])
    assert torch.equal(got, plain(x))
    with torch.no_grad():
        eager = model(x)
    assert float((got - eager).abs().max()) <= 2e-2 * float(eager.abs().max())


def test_tuner_is_asked_for_a16_exactly_where_a_can_be_stored_bf16():
    # the block's four products have producers that can round A to bf16 (the
    # LayerNorms, the attention, the MLP-up product): the tuner is asked to
    # time them reading bf16 A; a Linear on a graph input is not
    asked = []

    def cfg(graph, kernel, a16=False):
        asked.append((kernel.name, a16))
        return {"tile": 99, "splitk": 1}

    cfg.accepts_a16 = True
    torch.manual_seed(0)
    model = gpt2_init_(Block(128, 4, 16), seed=0).eval()
    kiln.compile(model, (torch.randn(16, 128),), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    assert len(asked) == 4 and all(a16 for _, a16 in asked), asked
    asked.clear()
    kiln.compile(torch.nn.Linear(128, 64), (torch.randn(16, 128),), device="cuda", matmul_precision="bf16",
                 gpu_matmul_config=cfg)
    assert asked and not any(a16 for _, a16 in asked), asked
    asked.clear()
    kiln.compile(model, (torch.randn(16, 128),), device="cuda", gpu_matmul_config=cfg)   # fp32: never
    assert asked and not any(a16 for _, a16 in asked), asked


def test_bf16_storage_needs_a_single_bf16_reader():
    # a LayerNorm output that is also a graph result stays fp32
    torch.manual_seed(1)
    ln = torch.nn.LayerNorm(128)
    lin = gpt2_init_(torch.nn.Linear(128, 64), seed=1)

    def fn(t):
        y = ln(t)
        return lin(y), y

    x = torch.randn(32, 128)
    c = kiln.compile(fn, (x,), device="cuda", matmul_precision="bf16",
                     gpu_matmul_config=lambda *_: {"tile": 99, "splitk": 1})
    assert not any("bf16" in l.summary.replace("tile 99 splitk 1 bf16", "") for l in c._exe.program.launches)


def test_bf16_attention_products_on_the_host():
    # a bf16 plan's attention (cfg[5] = 1) on the host: q, k rounded to bf16
    # for the scores (float64 sum, then the fp32 score and scale), the
    # normalised weights and v rounded to bf16 for the weighted sum
    class Attn(torch.nn.Module):
        def __init__(self, mask):
            super().__init__()
            self.register_buffer("mask", mask)

        def forward(self, q, k, v):
            return F.softmax((q @ k.transpose(-2, -1)) * 0.125 + self.mask, dim=-1) @ v

    T, d = 40, 64
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, T, d, generator=g) for _ in range(3))
    mask = torch.full((T, T), float("-inf")).triu(1)
    c = kiln.compile(Attn(mask), (q, k, v), device="cuda", matmul_precision="bf16")
    assert "products:bf16" in open(c.report.lowering["source"]).read()
    r = lambda a: oracle.bf16_round(np.asarray(a, np.float32)).astype(np.float64)
    s = (r(q.numpy()) @ r(k.numpy()).transpose(0, 2, 1)).astype(np.float32) * np.float32(0.125)
    s = s.astype(np.float64) + mask.numpy()
    e = np.exp(s - s.max(-1, keepdims=True))
    w = r((e / e.sum(-1, keepdims=True)).astype(np.float32))
    ref = w @ r(v.numpy())
    np.testing.assert_allclose(c(q, k, v).numpy().astype(np.float64), ref, rtol=1e-6, atol=1e-7)
    # decode shapes keep fp32 products
    c1 = kiln.compile(Attn(mask[:1]), (q[:, :1], k, v), device="cuda", matmul_precision="bf16")
    assert "products:bf16" not in open(c1.report.lowering["source"]).read()


def test_three_pass_attention_products_on_the_host(monkeypatch):
    # a three-pass plan's attention (cfg[5] = 2) on the host: q, k split into
    # bf16 hi = rn(x) and lo = rn(x - hi) for the scores (lo.hi + hi.lo + hi.hi
    # summed in float64, then the fp32 score and scale), the normalised
    # weights and v split the same way for the weighted sum
    from kiln.hip import lowering

    class Attn(torch.nn.Module):
        def __init__(self, mask):
            super().__init__()
            self.register_buffer("mask", mask)

        def forward(self, q, k, v):
            return F.softmax((q @ k.transpose(-2, -1)) * 0.125 + self.mask, dim=-1) @ v

    T, d = 40, 64
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, T, d, generator=g) for _ in range(3))
    mask = torch.full((T, T), float("-inf")).triu(1)
    # two query blocks of 32: under the library's grid bar, so fp32 products
    c0 = kiln.compile(Attn(mask), (q[:1], k[:1], v[:1]), device="cuda", allow_tf32=True)
    assert "products:bf16" not in open(c0.report.lowering["source"]).read()
    monkeypatch.setattr(lowering, "ATTN_X3_MIN_GROUPS", 0)
    c = kiln.compile(Attn(mask), (q, k, v), device="cuda", matmul_precision="bf16x3")
    assert "products:bf16x3" in open(c.report.lowering["source"]).read()

    def split(a):
        a = np.asarray(a, np.float32)
        hi = oracle.bf16_round(a)
        lo = oracle.bf16_round(np.where(np.isfinite(hi), a - hi, 0.0).astype(np.float32))
        return hi.astype(np.float64), lo.astype(np.float64)

    (qh, ql), (kh, kl), (vh, vl) = split(q.numpy()), split(k.numpy()), split(v.numpy())
    kt = lambda a: a.transpose(0, 2, 1)
    s = (ql @ kt(kh) + qh @ kt(kl) + qh @ kt(kh)).astype(np.float32) * np.float32(0.125)
    s = s.astype(np.float64) + mask.numpy()
    e = np.exp(s - s.max(-1, keepdims=True))
    wh, wl = split((e / e.sum(-1, keepdims=True)).astype(np.float32))
    ref = wl @ vh + wh @ vl + wh @ vh
    got = c(q, k, v).numpy().astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)
    # a dropped cross term would move the result by ~1e-3 of its scale
    assert np.abs(got - (wh @ vh)).max() > 1e-5


def test_pair_storage_in_three_pass_plans(monkeypatch):
    # allow_tf32 plans store as pair words (bf16 hi and lo halves of each
    # value) what only three-pass readers read: the LayerNorm outputs, the
    # attention's q, k, v and output, the MLP-up output; the host runs them as
    # fp32 storage, the same meaning
    from kiln.hip import lowering

    monkeypatch.setattr(lowering, "ATTN_X3_MIN_GROUPS", 0)
    T = 64
    model = gpt2_init_(Block(128, 4, T), seed=0).eval()
    x = torch.randn(T, 128)
    c = kiln.compile(model, (x,), device="cuda", allow_tf32=True)
    summaries = [l.summary for l in c._exe.program.launches]
    assert sum("A:pairs" in s for s in summaries) == 4, summaries
    assert any("qkv:pairs" in s and "out:pairs" in s for s in summaries), summaries
    assert sum("layernorm out:pairs" in s for s in summaries) == 2, summaries
    got = c(x)
    monkeypatch.setattr(lowering._Lowerer, "plan_pair_storage", lambda self: set())
    plain = kiln.compile(model, (x,), device="cuda", allow_tf32=True, plan_cache=False)
    assert not any("pairs" in l.summary for l in plain._exe.program.launches)
    assert torch.equal(got, plain(x))
    # bf16 and fp32 plans store nothing as pairs
    c16 = kiln.compile(model, (x * 1.0,), device="cuda", matmul_precision="bf16", plan_cache=False)
    assert not any("pairs" in l.summary for l in c16._exe.program.launches)
