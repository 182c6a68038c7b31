"""Parity of the bf16-input GEMM variant (matmul_precision="bf16").

The variant rounds both GEMM inputs to bf16 (round to nearest, ties to even:
the weights once, when the executable is built, the activations in the
kernel) and accumulates in fp32. Two checks, both written per test:
  * the exact reference of that computation: the C oracle's bf16 rounding of
    the inputs, then a float64 product. Only fp32 accumulation separates the
    kernel from it: |out - ref| <= 1e-4 * max|ref| (1e-4 relative to the
    output scale; a wrong rounding mode alone moves results by ~1e-3);
  * eager PyTorch fp32, at the north star's stated tolerance for bf16-input
    variants: rtol 2e-2, with atol 2e-2 * max|ref| for outputs near zero.
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kiln
import oracle
from kiln.hip import autotune
from models.transformer import Block, gpt2_init_

pytestmark = pytest.mark.gpu

EXACT = 1e-4          # relative to the output scale, against the rounded-input reference
# Through a chain of GEMMs the rounded-input reference is only approximate:
# the kernel's fp32 activations differ from the float64 reference's by ~1e-7,
# and an activation that close to a bf16 rounding boundary rounds to the other
# neighbour (a 2^-8 relative step in that input). 1e-3 of the output scale
# covers such flips and still fails a wrong rounding mode or a dropped term.
CHAINED = 1e-3
STATED = 2e-2         # against eager fp32


def r16(a):
    return oracle.bf16_round(np.asarray(a, np.float32)).astype(np.float64)


class _Batched(torch.nn.Module):
    """x @ w[b] * 0.5 over a constant batch of weights."""

    def __init__(self, w):
        super().__init__()
        self.w = torch.nn.Parameter(w)

    def forward(self, x):
        return torch.matmul(x, self.w) * 0.5


def close_to_scale(out, ref, tol):
    out, ref = np.asarray(out, np.float64), np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(out - ref).max() / scale
    assert err <= tol, f"max error {err:.2e} of the output scale > {tol:.0e}"


def stated(out, eager):
    eager = np.asarray(eager, np.float64)
    np.testing.assert_allclose(np.asarray(out, np.float64), eager, rtol=STATED,
                               atol=STATED * np.abs(eager).max())


@pytest.mark.parametrize("mnk", [(2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768),
                                 (128, 768, 3072), (1, 3072, 768)])
def test_config_gemm_sweep_bf16(mnk):
    m, n, k = mnk
    torch.manual_seed(0)
    lin = gpt2_init_(torch.nn.Linear(k, n), seed=1).eval()
    x = torch.randn(m, k)
    c = kiln.compile(lin, (x,), device="cuda", matmul_precision="bf16")
    assert c.report.lowering["precision"] == "bf16"
    out = c(x.cuda()).cpu().numpy()
    w, b = lin.weight.detach().numpy(), lin.bias.detach().numpy()
    ref = r16(x.numpy()) @ r16(w).T + b.astype(np.float64)
    close_to_scale(out, ref, EXACT)
    with torch.no_grad():
        stated(out, lin(x).numpy())


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.TILES) if autotune.PRECISION[t] == "bf16"])
def test_every_bf16_tile_configuration(tile):
    # ragged sizes (K = 61: not a multiple of 4 or 8), then interior tiles with
    # ragged edges; bias + residual epilogue; split-K 1 and 2; a deeper K
    # (several steps per wave for the small-M kernel)
    for m, n, k in ((77, 133, 61), (300, 452, 96), (128, 200, 768)):
        torch.manual_seed(tile)
        w = torch.randn(n, k) * 0.1
        b, r = torch.randn(n), torch.randn(m, n)
        model = torch.nn.Linear(k, n)
        with torch.no_grad():
            model.weight.copy_(w)
            model.bias.copy_(b)
        fn = lambda x, r: model(x) + r
        x = torch.randn(m, k)
        ref = r16(x.numpy()) @ r16(w.numpy()).T + b.numpy().astype(np.float64) + r.numpy()
        for splitk in (1, 2):
            c = kiln.compile(fn, (x, r), device="cuda", matmul_precision="bf16",
                             gpu_matmul_config=lambda *_: {"tile": tile, "splitk": splitk})
            close_to_scale(c(x, r).cpu().numpy(), ref, EXACT)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.K_CONTIGUOUS) if autotune.PRECISION[t] == "bf16"])
def test_k_contiguous_bf16_tiles_walk_several_tiles(tile):
    # the persistent K-contiguous kernel over the bf16 weight copy: more tiles
    # than CUs (each workgroup walks several, the next tile's first stages
    # issued before the current epilogue) with ragged edges, fewer steps than
    # ring stages and many steps; direct epilogue (bias + residual) and the
    # tape epilogue (a scale); repeated calls agree bit for bit. K is a
    # whole number of the tile's K steps (32 or 64 deep)
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    deep = autotune.TILES[tile][2]
    for m, n, k in ((4200, 2600, 64), (4200, 2600, 5 * deep), (300, 452, 768)):
        torch.manual_seed(m + k)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
        x, r = torch.randn(m, k), torch.randn(m, n)
        w, b = lin.weight.detach().numpy(), lin.bias.detach().numpy().astype(np.float64)
        prod = r16(x.numpy()) @ r16(w).T
        cases = ((lambda t, res: lin(t) + res, (x, r), prod + b + r.numpy()),
                 (lambda t, res: lin(t) * 0.5 - res, (x, r), (prod + b) * 0.5 - r.numpy()))
        for fn, args, ref in cases:
            c = kiln.compile(fn, args, device="cuda", cuda_graphs=False, matmul_precision="bf16",
                             gpu_matmul_config=cfg)
            assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
            out = c(*args)
            close_to_scale(out.cpu().numpy(), ref, EXACT)
            assert torch.equal(c(*args), out)
    # batched constant weights: each batch reads its own slice of the copy
    torch.manual_seed(tile)
    model = _Batched(torch.randn(3, 3 * deep, 50) * 0.1).eval()
    w = model.w.detach()
    x = torch.randn(3, 300, 3 * deep)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
    ref = np.stack([r16(x[i].numpy()) @ r16(w[i].numpy()) for i in range(3)]) * 0.5
    close_to_scale(c(x).cpu().numpy(), ref, EXACT)


@pytest.mark.parametrize("k, n, ln", [(768, 2304, True), (3072, 768, False), (64, 130, False), (16, 5, True)])
def test_bf16_gemv(k, n, ln):
    # one-row products with a constant weight run on the K-contiguous GEMV over
    # the bf16 [N][K] copy (x rounded to bf16, fp32 sums), with and without a
    # LayerNorm prologue (normalised in fp32, then rounded: CHAINED covers an
    # activation that lands on the other side of a bf16 rounding boundary)
    torch.manual_seed(k + n)
    lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
    layers = [torch.nn.LayerNorm(k)] if ln else []
    model = torch.nn.Sequential(*layers, lin).eval()
    x = 1.0 + torch.randn(1, k)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16")
    assert c.report.lowering["families"] == {"gemv": 1} and c.report.lowering["precision"] == "bf16"
    out = c(x.cuda()).cpu().numpy()
    xa = x.numpy().astype(np.float64)
    if ln:
        xa = (xa - xa.mean(-1, keepdims=True)) / np.sqrt(xa.var(-1, keepdims=True) + 1e-5)
    w, b = lin.weight.detach().numpy(), lin.bias.detach().numpy()
    ref = r16(xa) @ r16(w).T + b.astype(np.float64)
    close_to_scale(out, ref, CHAINED if ln else EXACT)
    with torch.no_grad():
        stated(out, model(x).numpy())
    for _ in range(2):
        assert np.array_equal(c(x.cuda()).cpu().numpy(), out)


def test_batched_constant_operand():
    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = torch.nn.Parameter(torch.randn(3, 24, 56))

        def forward(self, x):
            return torch.matmul(x, self.w)

    model = M().eval()
    x = torch.randn(3, 40, 24)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16")
    ref = np.matmul(r16(x.numpy()), r16(model.w.detach().numpy()))
    close_to_scale(c(x).cpu().numpy(), ref, EXACT)


def test_activation_product_stays_fp32():
    a, b = torch.randn(64, 32), torch.randn(32, 48)
    c = kiln.compile(lambda a, b: a @ b, (a, b), device="cuda", matmul_precision="bf16")
    np.testing.assert_allclose(c(a, b).cpu().numpy(), (a.double() @ b.double()).numpy(), rtol=1e-4, atol=1e-5)


def _bf16_reference_block(model):
    """float64 copy of the block whose Linear layers see bf16-rounded inputs
    and weights, and whose attention products see bf16-rounded q, k (scores)
    and softmax weights, v (weighted sum) - the computation the bf16 variant
    performs."""
    ref = copy.deepcopy(model).double()
    for mod in ref.modules():
        if isinstance(mod, torch.nn.Linear):
            with torch.no_grad():
                mod.weight.copy_(torch.from_numpy(r16(mod.weight.float().numpy())))
            mod.register_forward_pre_hook(
                lambda m, args: (torch.from_numpy(r16(args[0].float().numpy())),))
    rt = lambda t: torch.from_numpy(r16(t.float().numpy()))

    def attn(x):
        T, C = x.shape
        q, k, v = ref.c_attn(x).split(C, dim=1)
        hd = C // ref.nh
        q, k, v = (t.reshape(T, ref.nh, hd).transpose(0, 1) for t in (q, k, v))
        att = (rt(q) @ rt(k).transpose(-2, -1)) * (1.0 / hd ** 0.5) + ref.mask[:T, :T]
        y = (rt(F.softmax(att, dim=-1)) @ rt(v)).transpose(0, 1).reshape(T, C)
        return ref.c_proj(y)

    ref.attn = attn
    return ref


@pytest.mark.parametrize("T", [128, 512])
def test_gpt2_block_bf16(T):
    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16")
    out = c(x.cuda()).cpu().numpy()
    with torch.no_grad():
        ref = _bf16_reference_block(model)(x.double()).numpy()
        eager = model(x).numpy()
    close_to_scale(out, ref, CHAINED)
    stated(out, eager)


@pytest.mark.parametrize("queries", [16, 32])
def test_bf16_attention_output_on_both_query_blocks(queries, monkeypatch):
    # every product on a 64-deep bf16 configuration, so the attention (16 or
    # 32 queries per workgroup, ragged T) writes its head-merged output as
    # bf16 for the projection: the same bits as the plan with fp32 storage
    from kiln.hip import lowering

    monkeypatch.setattr(lowering, "ATTN_QUERIES", queries)
    T = 200
    torch.manual_seed(3)
    model = gpt2_init_(Block(768, 12, T), seed=3).eval()
    x = torch.randn(T, 768)
    cfg = lambda *_: {"tile": 99, "splitk": 1}
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    summaries = [l.summary for l in c._exe.program.launches]
    assert any("heads" in s and "out:bf16" in s for s in summaries), summaries
    # with 32 queries per workgroup the QKV product also writes q, k, v as
    # bf16 for the attention's bf16 products
    assert any("heads" in s and "qkv:bf16" in s for s in summaries) == (queries == 32), summaries
    xd = x.cuda()
    got = c(xd)
    monkeypatch.setattr(lowering._Lowerer, "plan_bf16_storage", lambda self: set())
    plain = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", gpu_matmul_config=cfg)
    assert not any("bf16" in s.split("bf16", 1)[-1] for s in [l.summary for l in plain._exe.program.launches])
    assert torch.equal(got, plain(xd))
    with torch.no_grad():
        eager = model(x).cuda()
    assert float((got - eager).abs().max()) <= STATED * float(eager.abs().max())


@pytest.mark.parametrize("T", [512, 2048])
def test_bf16_storage_gives_the_same_bits_on_the_block(T, monkeypatch):
    # the GPT-2 block with bf16 products (shipped table): producers whose only
    # reader is a 64-deep bf16 product store their outputs as bf16 (rounded
    # to nearest even, the rounding the product does at every fragment read),
    # so the result is bit for bit the one of the same plan with fp32 storage
    from kiln.hip import lowering

    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16")
    summaries = [l.summary for l in c._exe.program.launches]
    print(f"bf16 storage T={T}: " + " | ".join(summaries), flush=True)
    assert any("A:bf16" in s for s in summaries)
    xd = x.cuda()
    got = c(xd)
    monkeypatch.setattr(lowering._Lowerer, "plan_bf16_storage", lambda self: set())
    plain = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16", plan_cache=False)
    assert not any("A:bf16" in l.summary for l in plain._exe.program.launches)
    assert torch.equal(got, plain(xd))
    with torch.no_grad():
        eager = model(x).cuda()
    assert float((got - eager).abs().max()) <= STATED * float(eager.abs().max())


# -- attention with bf16 products ------------------------------------------------------------

@pytest.fixture(params=[0, 16, 32], ids=["q-auto", "q16", "q32"])
def queries(request, monkeypatch):
    """Queries per workgroup of the blocked kernel: the library's choice, or
    forced to 16 (attnbf_kernel) or 32 (attn_kernel with bf16 products)."""
    from kiln.hip import lowering

    monkeypatch.setattr(lowering, "ATTN_QUERIES", request.param)
    return request.param


class _Attn(torch.nn.Module):
    """softmax(q k^T * scale + mask) v over [B, T, D] inputs."""

    def __init__(self, mask=None, scale=0.125):
        super().__init__()
        self.scale = scale
        if mask is not None:
            self.register_buffer("mask", mask)
        else:
            self.mask = None

    def forward(self, q, k, v):
        s = (q @ k.transpose(-2, -1)) * self.scale
        if self.mask is not None:
            s = s + self.mask
        return F.softmax(s, dim=-1) @ v


def _bf16_attention_reference(q, k, v, scale, mask):
    """The unfused computation with bf16 products: q, k rounded for the
    scores, the normalised softmax weights and v rounded for the weighted sum,
    everything else float64."""
    s = r16(q.numpy()) @ r16(k.numpy()).transpose(0, 2, 1) * scale
    if mask is not None:
        s = s + mask.numpy().astype(np.float64)
    with np.errstate(invalid="ignore"):
        e = np.exp(s - s.max(-1, keepdims=True))
        p = e / e.sum(-1, keepdims=True)
    return r16(p.astype(np.float32)) @ r16(v.numpy())


def _check_bf16_attention(model, q, k, v, mask):
    c = kiln.compile(model, (q, k, v), device="cuda", matmul_precision="bf16")
    summaries = [l.summary for l in c._exe.program.launches]
    assert any("heads" in s and "products:bf16" in s for s in summaries), summaries
    got = c(q.cuda(), k.cuda(), v.cuda()).cpu().numpy().astype(np.float64)
    ref = _bf16_attention_reference(q, k, v, model.scale, mask)
    # the kernel rounds the running-max-relative probabilities, the reference
    # the normalised ones: each weight within 2^-9 of its value in both, so
    # the outputs agree to 2^-8 of the largest |v|
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    tol = 2.0 ** -8 * float(np.abs(v.numpy()).max()) + 1e-5
    err = float(np.abs(got[~nan] - ref[~nan]).max()) if (~nan).any() else 0.0
    assert err <= tol, f"max error {err:.2e} > {tol:.2e}"
    with torch.no_grad():
        eager = model(q, k, v).numpy().astype(np.float64)
    np.testing.assert_allclose(got[~nan], eager[~nan], rtol=STATED, atol=STATED * np.abs(eager[~nan]).max())
    return c


@pytest.mark.parametrize("T", [5, 77, 200, 512])
@pytest.mark.parametrize("d", [32, 64])
def test_bf16_attention_causal(T, d, queries):
    g = torch.Generator().manual_seed(T + d)
    q, k, v = (torch.randn(3, T, d, generator=g) for _ in range(3))
    mask = torch.full((T, T), float("-inf")).triu(1)
    _check_bf16_attention(_Attn(mask, 1 / d ** 0.5), q, k, v, mask)


@pytest.mark.parametrize("tq, tk", [(50, 90), (33, 7), (64, 64), (130, 300)])
def test_bf16_attention_cross(tq, tk, queries):
    g = torch.Generator().manual_seed(tq * 7 + tk)
    q, k, v = torch.randn(2, tq, 64, generator=g), torch.randn(2, tk, 64, generator=g), torch.randn(2, tk, 64, generator=g)
    _check_bf16_attention(_Attn(None, 0.125), q, k, v, None)


def test_bf16_attention_additive_mask_and_fully_masked_row(queries):
    tq, tk = 40, 70
    g = torch.Generator().manual_seed(11)
    q, k, v = torch.randn(2, tq, 64, generator=g), torch.randn(2, tk, 64, generator=g), torch.randn(2, tk, 64, generator=g)
    mask = torch.randn(tq, tk, generator=g)
    mask[torch.rand(tq, tk, generator=g) < 0.3] = float("-inf")
    mask[:, 0] = 0.0
    mask[7, :] = float("-inf")          # a fully masked row: NaN, as in eager
    _check_bf16_attention(_Attn(mask, 0.125), q, k, v, mask)


def test_bf16_attention_keeps_fp32_products_on_decode_shapes():
    g = torch.Generator().manual_seed(5)
    q, k, v = torch.randn(4, 1, 64, generator=g), torch.randn(4, 40, 64, generator=g), torch.randn(4, 40, 64, generator=g)
    c = kiln.compile(_Attn(None, 0.125), (q, k, v), device="cuda", matmul_precision="bf16")
    assert not any("products:bf16" in l.summary for l in c._exe.program.launches)
    with torch.no_grad():
        eager = _Attn(None, 0.125)(q, k, v)
    torch.testing.assert_close(c(q.cuda(), k.cuda(), v.cuda()).cpu(), eager, rtol=1e-4, atol=1e-5)
