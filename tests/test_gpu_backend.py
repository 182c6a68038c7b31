"""torch.compile(backend=kiln.backend) on the MI355X: results match eager
PyTorch at the reference's tolerances (rtol 1e-4, atol 1e-5;
tests/test_compile.py:108-116 there) - and the GPT-2 block also the float64
C oracle - and weights stay runtime inputs."""

import numpy as np
import pytest
import torch

import kiln
import oracle
from models.transformer import Block, gpt2_init_

pytestmark = pytest.mark.gpu


def _fresh():
    kiln.stats.update(compiled=0, fallback=0)
    torch._dynamo.reset()


def test_linear_gelu_compiles_for_the_gpu():
    _fresh()
    model = torch.nn.Sequential(torch.nn.Linear(8, 16), torch.nn.GELU()).eval().cuda()
    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)
    x = torch.randn(4, 8, device="cuda")
    with torch.no_grad():
        torch.testing.assert_close(compiled(x), model(x), rtol=1e-4, atol=1e-5)
    assert kiln.stats == {"compiled": 1, "fallback": 0}


def test_weight_updates_are_seen():
    _fresh()
    model = torch.nn.Linear(64, 32).eval().cuda()
    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)
    x = torch.randn(16, 64, device="cuda")
    with torch.no_grad():
        torch.testing.assert_close(compiled(x), model(x), rtol=1e-4, atol=1e-5)
        model.weight.add_(0.5)
        torch.testing.assert_close(compiled(x), model(x), rtol=1e-4, atol=1e-5)
    assert kiln.stats["compiled"] == 1


@pytest.mark.parametrize("T", [128, 512])
def test_gpt2_block_compiles_for_the_gpu(T):
    _fresh()
    torch.manual_seed(0)
    model = gpt2_init_(Block(768, 12, T), seed=0).eval().cuda()
    compiled = torch.compile(model, backend=kiln.backend, dynamic=False)
    x = torch.randn(T, 768, device="cuda")
    with torch.no_grad():
        got = compiled(x)
        torch.testing.assert_close(got, model(x), rtol=1e-4, atol=1e-5)
    assert kiln.stats == {"compiled": 1, "fallback": 0}
    # and against the float64 C oracle of the block
    params = {k: v.detach().cpu().numpy() for k, v in model.state_dict().items()}
    ref = oracle.block(x.cpu().numpy(), params, 12)
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-4, atol=1e-5)
