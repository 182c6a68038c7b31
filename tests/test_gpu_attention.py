"""Parity of the fused attention family (kiln.hip.attention + kh_attn.hip).

The fused kernel must give what the five-kernel path gives: every case is
compared with the float64 oracle (interpreter over the imported graph, or the
C oracle for the GPT-2 block) and with eager PyTorch fp32 at the fp32
tolerance (rtol 1e-4, atol 1e-5), and checks that the fused launch was used.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kiln
import oracle
from kiln.hip import lib as kl
from models.transformer import Block, gpt2_init_
from oracle import interp
from test_gpu import ATOL, RTOL, as_tuple, imported

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[0, 16, 32], ids=["q-auto", "q16", "q32"])
def queries(request, monkeypatch):
    """Queries per workgroup of the blocked kernel: the library's choice, or
    forced to 16 (attn16_kernel) or 32."""
    from kiln.hip import lowering

    monkeypatch.setattr(lowering, "ATTN_QUERIES", request.param)
    return request.param


def n_attention(compiled):
    return sum(1 for l in compiled._exe.program.launches if l.family == kl.FAM_ATTN)


def compare(fn, *xs, fused=1, rtol=RTOL, atol=ATOL, **flags):
    compiled = kiln.compile(fn, xs, device="cuda", **flags)
    assert n_attention(compiled) == fused, compiled._exe.program.source
    ref = interp.run(imported(fn, xs), *[x.numpy() for x in xs])
    with torch.no_grad():
        eager = as_tuple(fn(*xs))
    got = as_tuple(compiled(*xs))
    for a, r, e in zip(got, ref, eager):
        np.testing.assert_allclose(a.cpu().numpy().astype(np.float64), r, rtol=rtol, atol=atol)
        torch.testing.assert_close(a.cpu(), e, rtol=rtol, atol=atol, equal_nan=True)
    return compiled


class Attn(torch.nn.Module):
    """softmax(q k^T scale + mask) v over [B, T, D] inputs, heads merged into [Tq, B*D]."""

    def __init__(self, mask=None, scale=0.125, divide=False, merge=True):
        super().__init__()
        self.scale, self.divide, self.merge = scale, divide, merge
        if mask is not None:
            self.register_buffer("mask", mask)
        else:
            self.mask = None

    def forward(self, q, k, v):
        s = q @ k.transpose(-2, -1)
        s = s / self.scale if self.divide else s * self.scale
        if self.mask is not None:
            s = s + self.mask
        o = F.softmax(s, dim=-1) @ v
        if self.merge:
            o = o.transpose(0, 1).contiguous().view(q.shape[1], -1)
        return o


def qkv(b, tq, tk, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, tq, d, generator=g), torch.randn(b, tk, d, generator=g),
            torch.randn(b, tk, d, generator=g))


@pytest.mark.parametrize("T", [1, 5, 32, 77, 128, 200])
@pytest.mark.parametrize("d", [32, 64])
def test_causal(T, d, queries):
    mask = torch.full((T, T), float("-inf")).triu(1)
    c = compare(Attn(mask, scale=1 / math.sqrt(d)), *qkv(3, T, T, d, seed=T))
    assert "causal" in c._exe.program.source


@pytest.mark.parametrize("tq, tk", [(1, 40), (50, 90), (64, 64), (33, 7)])
def test_no_mask_cross_attention(tq, tk, queries):
    compare(Attn(None, scale=0.125), *qkv(2, tq, tk, 64, seed=tq + tk))


@pytest.mark.parametrize("tq, tk", [(1, 1), (1, 40), (3, 9), (4, 64), (2, 65)])
@pytest.mark.parametrize("d", [32, 64])
@pytest.mark.parametrize("masked", [False, True])
def test_few_query_rows(tq, tk, d, masked):
    # decode shapes (up to 4 queries over up to 64 keys) run one wave per query
    # row; (2, 65) is just past that and runs the MFMA kernel. The additive
    # mask has -inf entries and, with several queries, one fully masked row
    # (NaN, as in eager)
    mask = None
    if masked:
        g = torch.Generator().manual_seed(tq * 100 + tk)
        mask = torch.randn(tq, tk, generator=g)
        mask[torch.rand(tq, tk, generator=g) < 0.3] = float("-inf")
        mask[:, 0] = 0.0
        if tq > 1:
            mask[1, :] = float("-inf")
    compare(Attn(mask, scale=8.0, divide=True, merge=False), *qkv(3, tq, tk, d, seed=tq + tk + d))


class AttnProj(torch.nn.Module):
    """One query's attention over tk keys, heads merged, then a Linear (decode)."""

    def __init__(self, heads, d, mask=None, divide=False):
        super().__init__()
        self.attn = Attn(mask, scale=8.0 if divide else 0.125, divide=divide)
        self.proj = torch.nn.Linear(heads * d, 48)

    def forward(self, q, k, v):
        return self.proj(self.attn(q, k, v))


@pytest.mark.parametrize("tk, d, masked, prec", [(1, 64, False, "fp32"), (40, 64, True, "fp32"),
                                                 (9, 32, False, "fp32"), (64, 64, True, "bf16"),
                                                 (7, 32, True, "bf16"), (65, 64, False, "fp32")])
def test_decode_attention_as_gemv_prologue(tk, d, masked, prec):
    # one query over at most 64 keys feeding a GEMV: the GEMV computes the
    # attention for the K values it loads and no attention kernel runs
    # (65 keys: past that, the attention launch stays)
    heads = 4
    mask = None
    if masked:
        g = torch.Generator().manual_seed(tk)
        mask = torch.randn(1, tk, generator=g)
        mask[torch.rand(1, tk, generator=g) < 0.3] = float("-inf")
        mask[:, 0] = 0.0
    model = AttnProj(heads, d, mask, divide=tk % 2 == 1).eval()
    q, k, v = qkv(heads, 1, tk, d, seed=tk + d)
    fused = tk <= 64
    if prec == "fp32":
        c = compare(model, q, k, v, fused=0 if fused else 1)
    else:
        c = kiln.compile(model, (q, k, v), device="cuda", matmul_precision=prec)
        assert n_attention(c) == 0
        with torch.no_grad():
            eager = model(q, k, v)
        got = c(q, k, v).cpu()
        torch.testing.assert_close(got, eager, rtol=2e-2, atol=2e-2 * eager.abs().max().item())
    assert ("prologue: attention" in c._exe.program.source) == fused
    first = c(q, k, v)
    for _ in range(2):
        assert torch.equal(c(q, k, v), first)


def test_divided_scale_and_no_head_merge(queries):
    c = compare(Attn(None, scale=8.0, divide=True, merge=False), *qkv(4, 70, 70, 64, seed=3))
    assert "scores / 8" in c._exe.program.source


def test_additive_mask(queries):
    g = torch.Generator().manual_seed(7)
    mask = torch.randn(45, 60, generator=g)
    mask[torch.rand(45, 60, generator=g) < 0.3] = float("-inf")
    mask[:, 0] = 0.0                      # every row keeps a finite score
    c = compare(Attn(mask), *qkv(3, 45, 60, 32, seed=1))
    assert "additive mask" in c._exe.program.source


def test_fully_masked_rows_are_nan_as_in_eager(queries):
    mask = torch.zeros(20, 20)
    mask[3, :] = float("-inf")
    mask[11, :] = float("-inf")
    q, k, v = qkv(2, 20, 20, 64, seed=5)
    fn = Attn(mask, merge=False)
    compiled = kiln.compile(fn, (q, k, v), device="cuda")
    assert n_attention(compiled) == 1
    with torch.no_grad():
        eager = fn(q, k, v)
    got = compiled(q, k, v).cpu()
    assert torch.isnan(eager[:, [3, 11]]).all()
    torch.testing.assert_close(got, eager, rtol=RTOL, atol=ATOL, equal_nan=True)


def test_unsupported_head_dim_is_not_fused():
    compare(Attn(None, scale=0.25), *qkv(2, 24, 24, 16, seed=2), fused=0)


def test_fusion_can_be_turned_off():
    compare(Attn(None), *qkv(2, 40, 40, 64, seed=4), fused=0, fused_attention=False)


@pytest.mark.parametrize("T", [1, 77, 128, 512])
def test_block_uses_one_attention_launch(T):
    model = gpt2_init_(Block(768, 12, T), seed=T).eval()
    x = torch.randn(T, 768, generator=torch.Generator().manual_seed(T + 1))
    c = kiln.compile(model, (x,), device="cuda")
    # at T = 1 both LayerNorms run as the prologue of the qkv / fc GEMV
    # at T = 1 the attention runs as the prologue of the c_proj GEMV
    # at T > 1 a LayerNorm feeding a small-M GEMM runs as that GEMM's prologue
    n_pro = sum("prologue: layernorm" in l.summary for l in c._exe.program.launches)
    assert (c.report.lowering["launches"], n_attention(c)) == ((4, 0) if T == 1 else (7 - n_pro, 1))
    # the scores never get arena memory: the peak is the MLP's (768 + 768 + 3072) T floats
    assert c.report.arena_bytes == 4 * 4608 * T
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    want = oracle.block(x.numpy(), params, 12)
    got = c(x).cpu()
    np.testing.assert_allclose(got.numpy().astype(np.float64), want, rtol=RTOL, atol=ATOL)
    with torch.no_grad():
        torch.testing.assert_close(got, model(x), rtol=RTOL, atol=ATOL)


def test_fused_matches_unfused_at_1024():
    T = 1024
    model = gpt2_init_(Block(768, 12, T), seed=9).eval().cuda()
    x = torch.randn(T, 768, device="cuda")
    fused = kiln.compile(model, (x,), device="cuda")
    plain = kiln.compile(model, (x,), device="cuda", fused_attention=False)
    assert n_attention(fused) == 1 and n_attention(plain) == 0
    torch.testing.assert_close(fused(x), plain(x), rtol=RTOL, atol=ATOL)
