"""Persistent GEMV chains on the GPU: consecutive one-row matmuls (decode)
run as one launch whose stages hand their outputs over as (value, epoch)
words. Checked against the oracle and against the same plan run launch by
launch (the default), over repeated calls (each call a new epoch), new
inputs, hipGraph replay and direct runs, fp32 and bf16 weights, and with
stage outputs that are also plan outputs in the middle of the chain. Every
case also checks that no bounded wait inside the chain gave up."""

import copy

import numpy as np
import pytest
import torch

import kiln
import oracle
from models.transformer import Stack, gpt2_init_
from test_gpu import ATOL, RTOL, _LayerTaps

pytestmark = pytest.mark.gpu


def _stack(layers, d, heads, seed=0):
    torch.manual_seed(seed)
    return gpt2_init_(Stack(layers, d, heads, 1), seed=seed).eval()


def _oracle_stack(model, x, heads):
    h = x.numpy().astype(np.float64)
    for blk in model.blocks:
        h = oracle.block(h, {k: v.numpy() for k, v in blk.state_dict().items()}, heads)
    sd = model.ln_f.state_dict()
    return oracle.layernorm(h, sd["weight"].numpy(), sd["bias"].numpy())


def _chained(model, x, **flags):
    c = kiln.compile(model, (x,), device="cuda", gemv_chains=True, **flags)
    plain = kiln.compile(model, (x,), device="cuda", **flags)
    return c, plain


@pytest.mark.parametrize("layers, d, heads", [(12, 768, 12), (2, 128, 4), (3, 256, 4)])
@pytest.mark.parametrize("graphs", [True, False], ids=["graph", "direct"])
def test_decode_stack_runs_as_one_chain(layers, d, heads, graphs):
    model = _stack(layers, d, heads)
    x = torch.randn(1, d)
    print(f"chain: stack layers={layers} d={d} heads={heads} graphs={graphs}", flush=True)
    c, plain = _chained(model, x, cuda_graphs=graphs)
    assert c.report.lowering["gemv_chains"] == [(0, 4 * layers)]
    assert c.report.lowering["kernel_launches"] == 2          # the chain, then the final LayerNorm
    assert plain.report.lowering["kernel_launches"] == 4 * layers + 1
    xd = x.cuda()
    got = c(xd)
    np.testing.assert_allclose(got.cpu().numpy(), _oracle_stack(model, x, heads), rtol=RTOL, atol=ATOL)
    torch.testing.assert_close(got, plain(xd), rtol=RTOL, atol=ATOL)
    for _ in range(4):
        assert torch.equal(c(xd), got)                        # every call a new epoch, same result
    for seed in range(3):
        torch.manual_seed(100 + seed)
        x2 = torch.randn(1, d, device="cuda") * (1 + seed)
        torch.testing.assert_close(c(x2), plain(x2), rtol=RTOL, atol=ATOL)
    assert c._exe.plan.chain_timeouts() == 0


def test_decode_stack_chain_with_bf16_weights():
    model = _stack(4, 768, 12)
    x = torch.randn(1, 768)
    c, plain = _chained(model, x, matmul_precision="bf16")
    assert c.report.lowering["gemv_chains"] == [(0, 16)]
    xd = x.cuda()
    got, ref = c(xd), plain(xd)
    # the same bf16 arithmetic (x rounded to bf16 at the product, fp32 sums);
    # summation order differs, so a bf16 rounding of x can flip
    scale = float(ref.abs().max())
    assert float((got - ref).abs().max()) <= 2e-3 * scale
    with torch.no_grad():
        eager = model(x).cuda()
    assert float((got - eager).abs().max()) <= 2e-2 * float(eager.abs().max())
    assert torch.equal(c(xd), got)
    assert c._exe.plan.chain_timeouts() == 0


def test_chain_with_plan_outputs_inside():
    # every block's output is also a graph result: stages in the middle of
    # the chain store to plan outputs, and the next stage reads them through
    # the hand-over words
    model = _stack(3, 256, 4)
    taps = _LayerTaps(model).eval()
    x = torch.randn(1, 256)
    c, plain = _chained(taps, x)
    assert c.report.lowering["gemv_chains"] == [(0, 12)]
    xd = x.cuda()
    got, ref = c(xd), plain(xd)
    with torch.no_grad():
        eager = copy.deepcopy(taps).cuda()(xd)
    for g, r, e in zip(got, ref, eager):
        torch.testing.assert_close(g, r, rtol=RTOL, atol=ATOL)
        torch.testing.assert_close(g, e, rtol=RTOL, atol=ATOL)
    assert c._exe.plan.chain_timeouts() == 0


def test_chain_launch_timing_covers_every_launch():
    # kh_plan_time of one launch runs that launch alone; of the whole plan
    # (index -1), the chain's one launch
    model = _stack(2, 768, 12)
    x = torch.randn(1, 768)
    c = kiln.compile(model, (x,), device="cuda", gemv_chains=True)
    per_launch = c.profile(x.cuda(), iters=5)
    assert len(per_launch) == 9 and all(row[-1] > 0 for row in per_launch)
    assert torch.equal(c(x.cuda()), c(x.cuda()))
    assert c._exe.plan.chain_timeouts() == 0


def test_chain_give_up_is_loud():
    # The host makes every bounded wait inside the chain give up at once (a
    # negative spin bound: no wait is attempted, every kernel exits normally).
    # Each workgroup then stores NaN as the outputs it owes, so everything
    # computed from the chain is NaN, and the runtime's check raises; with
    # the bound restored the plan is correct again.
    model = _stack(2, 128, 4)
    x = torch.randn(1, 128)
    c, plain = _chained(model, x)
    exe = c._exe
    assert exe.has_chains
    xd = x.cuda()
    ref = plain(xd)
    torch.testing.assert_close(c(xd), ref, rtol=RTOL, atol=ATOL)   # the first call's check passes
    exe.plan.set_chain_spin(-1)
    out = exe._direct(exe._prepare([xd]))[0]
    torch.cuda.synchronize()
    assert bool(torch.isnan(out).all())
    with pytest.raises(RuntimeError, match="gave up"):
        exe.check_chains()
    exe.plan.set_chain_spin(2_000_000)
    torch.testing.assert_close(exe._direct(exe._prepare([xd]))[0], ref, rtol=RTOL, atol=ATOL)
    exe.check_chains()                                           # nothing new gave up
    torch.testing.assert_close(c(xd), ref, rtol=RTOL, atol=ATOL)


def test_debug_mode_runs_a_chained_plan_launch_by_launch():
    # debug builds run every launch on its own (poison and canary checks
    # between launches), so the persistent chain is not used: a chain whose
    # waits would all give up changes nothing there
    model = _stack(2, 128, 4)
    x = torch.randn(1, 128)
    c, plain = _chained(model, x, debug=True)
    c._exe.plan.set_chain_spin(-1)
    xd = x.cuda()
    torch.testing.assert_close(c(xd), plain(xd), rtol=RTOL, atol=ATOL)
    assert c._exe.plan.chain_timeouts() == 0


def test_chain_give_up_raises_at_first_call():
    model = _stack(2, 128, 4)
    x = torch.randn(1, 128)
    c = kiln.compile(model, (x,), device="cuda", gemv_chains=True, cuda_graphs=False)
    c._exe.plan.set_chain_spin(-1)
    with pytest.raises(RuntimeError, match="gave up"):
        c(x.cuda())
