"""Parity of the three-pass bf16 GEMM (allow_tf32=True, or
matmul_precision="bf16x3"): gfx950 has no TF32 matrix instruction, so the
option the reference exposes for its GPU GEMMs (reference api.py Options,
test_gpu.py:116-122 at rtol 1e-2) maps to this variant here.

Both GEMM inputs split into bf16 hi = rn(x) and lo = rn(x - hi) (round to
nearest, ties to even; the weights once, when the executable is built, the
activations in the kernel), and a.b = a_lo.b_hi + a_hi.b_lo + a_hi.b_hi with
fp32 accumulation. Two checks, both written per test:
  * the exact reference of that computation - the C oracle's bf16 rounding
    for the splits, then float64 products: |out - ref| <= 1e-5 * max|ref|
    (only fp32 accumulation separates them; a dropped cross term moves
    results by ~1e-3 of the output scale);
  * float64 products of the unsplit fp32 inputs: |out - ref| <= 5e-5 *
    max|ref| (the dropped lo.lo term and the rounding of lo are ~2^-16 of
    each product; measured at most 8e-6 of the scale on these shapes).
"""

import numpy as np
import pytest
import torch

import kiln
import oracle
from kiln.hip import autotune
from models.transformer import Block, gpt2_init_

pytestmark = pytest.mark.gpu

SPLIT_EXACT = 1e-5    # against the three-product reference, relative to the output scale
FP32_CLASS = 5e-5     # against float64 of the unsplit inputs, relative to the output scale


def split(a):
    a = np.asarray(a, np.float32)
    hi = oracle.bf16_round(a)
    lo = oracle.bf16_round(np.where(np.isfinite(hi), a - hi, 0.0).astype(np.float32))
    return hi.astype(np.float64), lo.astype(np.float64)


def three_pass(x, w_kn):
    xh, xl = split(x)
    wh, wl = split(w_kn)
    return xl @ wh + xh @ wl + xh @ wh


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


@pytest.mark.parametrize("mnk", [(2048, 3072, 768), (128, 2304, 768), (128, 768, 768), (128, 3072, 768),
                                 (128, 768, 3072), (1, 3072, 768)])
def test_config_gemm_sweep_bf16x3(mnk):
    m, n, k = mnk
    torch.manual_seed(0)
    lin = gpt2_init_(torch.nn.Linear(k, n), seed=1).eval()
    x = torch.randn(m, k)
    c = kiln.compile(lin, (x,), device="cuda", allow_tf32=True)
    assert c.report.lowering["precision"] == "bf16x3"
    out = c(x.cuda()).cpu().numpy()
    w, b = lin.weight.detach().numpy(), lin.bias.detach().numpy().astype(np.float64)
    close_to_scale(out, three_pass(x.numpy(), w.T) + b, SPLIT_EXACT)
    close_to_scale(out, x.numpy().astype(np.float64) @ w.T.astype(np.float64) + b, FP32_CLASS)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.TILES) if autotune.PRECISION[t] == "bf16x3"])
def test_every_bf16x3_tile_configuration(tile):
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
        ref = three_pass(x.numpy(), w.numpy().T) + b.numpy().astype(np.float64) + r.numpy()
        for splitk in (1, 2):
            c = kiln.compile(fn, (x, r), device="cuda", matmul_precision="bf16x3",
                             gpu_matmul_config=lambda *_: {"tile": tile, "splitk": splitk})
            close_to_scale(c(x, r).cpu().numpy(), ref, SPLIT_EXACT)


@pytest.mark.parametrize("tile", [t for t in sorted(autotune.K_CONTIGUOUS) if autotune.PRECISION[t] == "bf16x3"])
def test_k_contiguous_bf16x3_tiles_walk_several_tiles(tile):
    # the persistent K-contiguous kernel over the three-pass copy (hi and lo
    # rows per stage): more tiles than CUs with ragged edges, short and long
    # K; direct and tape epilogues; repeated calls agree bit for bit
    cfg = lambda *_: {"tile": tile, "splitk": 1}
    for m, n, k in ((4200, 2600, 64), (300, 452, 768)):
        torch.manual_seed(m + k)
        lin = gpt2_init_(torch.nn.Linear(k, n), seed=k).eval()
        x, r = torch.randn(m, k), torch.randn(m, n)
        w, b = lin.weight.detach().numpy(), lin.bias.detach().numpy().astype(np.float64)
        prod = three_pass(x.numpy(), w.T)
        cases = ((lambda t, res: lin(t) + res, (x, r), prod + b + r.numpy()),
                 (lambda t, res: lin(t) * 0.5 - res, (x, r), (prod + b) * 0.5 - r.numpy()))
        for fn, args, ref in cases:
            c = kiln.compile(fn, args, device="cuda", cuda_graphs=False, matmul_precision="bf16x3",
                             gpu_matmul_config=cfg)
            assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
            out = c(*args)
            close_to_scale(out.cpu().numpy(), ref, SPLIT_EXACT)
            assert torch.equal(c(*args), out)
    # batched constant weights: each batch reads its own slice of the copy
    torch.manual_seed(tile)
    model = _Batched(torch.randn(3, 96, 50) * 0.1).eval()
    w = model.w.detach()
    x = torch.randn(3, 300, 96)
    c = kiln.compile(model, (x,), device="cuda", matmul_precision="bf16x3", gpu_matmul_config=cfg)
    assert f"tile {tile} splitk 1" in c._exe.program.launches[0].summary
    ref = np.stack([three_pass(x[i].numpy(), w[i].numpy()) for i in range(3)]) * 0.5
    close_to_scale(c(x).cpu().numpy(), ref, SPLIT_EXACT)


@pytest.mark.parametrize("T", [128, 512, 2048])
def test_gpt2_block_allow_tf32(T):
    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda", allow_tf32=True)
    assert c.report.lowering["precision"] == "bf16x3"
    out = c(x.cuda()).cpu().numpy()
    with torch.no_grad():
        ref = model.double()(x.double()).numpy()
    close_to_scale(out, ref, FP32_CLASS)


# -- attention with three-pass products ---------------------------------------------------------
# Three-pass plans run attention's two products on the same splits: q, k for
# the scores, the probabilities and v for the weighted sum (hi.lo + lo.hi +
# hi.hi, fp32 accumulation, scale, mask and softmax fp32), on the 32-query
# kernel where its grid has at least lowering.ATTN_X3_MIN_GROUPS workgroups
# (the tests below lower that bar to 0 to reach ragged and small shapes).

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
        return torch.softmax(s, dim=-1) @ v


def _three_pass_attention_reference(q, k, v, scale, mask):
    """The unfused computation with three-pass products: the scores from the
    splits of q and k, the normalised softmax weights (fp32) and v split for
    the weighted sum, everything else float64."""
    qh, ql = split(q.numpy())
    kh, kl = split(k.numpy())
    kt = lambda a: a.transpose(0, 2, 1)
    s = (ql @ kt(kh) + qh @ kt(kl) + qh @ kt(kh)) * scale
    if mask is not None:
        s = s + mask.numpy().astype(np.float64)
    with np.errstate(invalid="ignore"):
        e = np.exp(s - s.max(-1, keepdims=True))
        p = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    ph, pl = split(p)
    vh, vl = split(v.numpy())
    return pl @ vh + ph @ vl + ph @ vh


@pytest.fixture
def x3_everywhere(monkeypatch):
    from kiln.hip import lowering

    monkeypatch.setattr(lowering, "ATTN_X3_MIN_GROUPS", 0)


def _check_x3_attention(model, q, k, v, mask, expect=True):
    c = kiln.compile(model, (q, k, v), device="cuda", allow_tf32=True)
    summaries = [l.summary for l in c._exe.program.launches]
    assert any("heads" in s for s in summaries), summaries
    assert any("products:bf16x3" in s for s in summaries) == expect, summaries
    got = c(q.cuda(), k.cuda(), v.cuda()).cpu().numpy().astype(np.float64)
    nan = np.isnan(_three_pass_attention_reference(q, k, v, model.scale, mask))
    assert np.array_equal(np.isnan(got), nan)
    # the kernel splits the running-max-relative probabilities, the reference
    # the normalised ones: each weight's split is within ~2^-16 of it in both
    ref = _three_pass_attention_reference(q, k, v, model.scale, mask)
    tol = 2.0 ** -15 * float(np.abs(v.numpy()).max()) + 1e-6
    err = float(np.abs(got[~nan] - ref[~nan]).max()) if (~nan).any() else 0.0
    assert err <= tol, f"max error {err:.2e} > {tol:.2e}"
    # and fp32-class against float64 of the unsplit inputs
    with torch.no_grad():
        f64 = model.double()(q.double(), k.double(), v.double()).numpy()
    model.float()
    close_to_scale(got[~nan], f64[~nan], FP32_CLASS)
    return c


@pytest.mark.parametrize("T", [5, 77, 200, 512])
@pytest.mark.parametrize("d", [32, 64])
def test_x3_attention_causal(T, d, x3_everywhere):
    g = torch.Generator().manual_seed(T + d)
    q, k, v = (torch.randn(3, T, d, generator=g) for _ in range(3))
    mask = torch.full((T, T), float("-inf")).triu(1)
    _check_x3_attention(_Attn(mask, 1 / d ** 0.5), q, k, v, mask)


@pytest.mark.parametrize("tq, tk", [(50, 90), (33, 7), (64, 64), (130, 300)])
def test_x3_attention_cross(tq, tk, x3_everywhere):
    g = torch.Generator().manual_seed(tq * 7 + tk)
    q, k, v = torch.randn(2, tq, 64, generator=g), torch.randn(2, tk, 64, generator=g), torch.randn(2, tk, 64, generator=g)
    _check_x3_attention(_Attn(None, 0.125), q, k, v, None)


def test_x3_attention_additive_mask_and_fully_masked_row(x3_everywhere):
    tq, tk = 40, 70
    g = torch.Generator().manual_seed(11)
    q, k, v = torch.randn(2, tq, 64, generator=g), torch.randn(2, tk, 64, generator=g), torch.randn(2, tk, 64, generator=g)
    mask = torch.randn(tq, tk, generator=g)
    mask[torch.rand(tq, tk, generator=g) < 0.3] = float("-inf")
    mask[:, 0] = 0.0
    mask[7, :] = float("-inf")          # a fully masked row: NaN, as in eager
    _check_x3_attention(_Attn(mask, 0.125), q, k, v, mask)


@pytest.mark.parametrize("heads, T, expect", [(12, 512, True), (12, 1024, True), (12, 256, False), (3, 2048, True)])
def test_x3_attention_by_grid_size(heads, T, expect):
    # the library default: three-pass products from 192 query blocks of 32 on
    # (eight waves per workgroup at T = 1024, four at 512 and 2048), fp32
    # products on the 16-query kernel below
    g = torch.Generator().manual_seed(heads + T)
    q, k, v = (torch.randn(heads, T, 64, generator=g) for _ in range(3))
    mask = torch.full((T, T), float("-inf")).triu(1)
    _check_x3_attention(_Attn(mask, 0.125), q, k, v, mask, expect=expect)


def test_x3_attention_keeps_fp32_products_on_decode_shapes(x3_everywhere):
    g = torch.Generator().manual_seed(5)
    q, k, v = torch.randn(4, 1, 64, generator=g), torch.randn(4, 40, 64, generator=g), torch.randn(4, 40, 64, generator=g)
    c = kiln.compile(_Attn(None, 0.125), (q, k, v), device="cuda", allow_tf32=True)
    assert not any("products:bf16" in l.summary for l in c._exe.program.launches)
    with torch.no_grad():
        eager = _Attn(None, 0.125)(q, k, v)
    torch.testing.assert_close(c(q.cuda(), k.cuda(), v.cuda()).cpu(), eager, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("T", [256, 512, 1024, 2048])
def test_pair_storage_gives_the_same_bits_on_the_block(T, monkeypatch):
    # the GPT-2 block with allow_tf32 (shipped table): producers whose only
    # reader splits each value into bf16 hi and lo halves (the three-pass
    # products' A operands, the three-pass attention's q, k, v) store those
    # halves as pair words, so the result is bit for bit the one of the same
    # plan with fp32 storage
    from kiln.hip import lowering

    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval()
    x = torch.randn(T, 768)
    c = kiln.compile(model, (x,), device="cuda", allow_tf32=True)
    summaries = [l.summary for l in c._exe.program.launches]
    print(f"pair storage T={T}: " + " | ".join(summaries), flush=True)
    assert sum("A:pairs" in s for s in summaries) == 4
    assert any("qkv:pairs" in s for s in summaries) == (T >= 512)
    xd = x.cuda()
    got = c(xd)
    monkeypatch.setattr(lowering._Lowerer, "plan_pair_storage", lambda self: set())
    plain = kiln.compile(model, (x,), device="cuda", allow_tf32=True, plan_cache=False)
    assert not any("pairs" in l.summary for l in plain._exe.program.launches)
    assert torch.equal(got, plain(xd))
    # non-finite activations too (a non-finite hi half keeps its lo half 0)
    xn = xd.clone()
    xn[3, 5], xn[11, 0] = float("inf"), float("-inf")
    xn[7] = float("nan")
    torch.testing.assert_close(c(xn), plain(xn), rtol=0, atol=0, equal_nan=True)
    with torch.no_grad():
        f64 = model.double()(x.double()).numpy()
    model.float()
    close_to_scale(got.cpu().numpy(), f64, FP32_CLASS)
