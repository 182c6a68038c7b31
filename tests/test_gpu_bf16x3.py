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


@pytest.mark.parametrize("T", [128, 512])
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
