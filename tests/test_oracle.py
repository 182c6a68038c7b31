"""Pin the oracle before trusting it (CPU only).

Each oracle function is checked against something independent of its own
formula: PyTorch float64 library routines (F.gelu, F.layer_norm, F.softmax,
torch.matmul, the Block module itself), closed forms and invariants (softmax
rows sum to 1 and are shift-invariant; LayerNorm output has mean 0 and
variance var/(var+eps); GELU's limits and symmetry gelu(x) - gelu(-x) = x;
matmul against the identity and a rank-1 outer product), and brute force on
tiny inputs. A plausible mistake (dropped epsilon, wrong reduction axis,
transposed operand, wrong GELU constant, missing causal mask) fails at
least one test.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import interp
from models.transformer import Block, gpt2_init_

rng = np.random.default_rng(1234)


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


@pytest.mark.parametrize("approx", ["none", "tanh"])
def test_gelu_matches_torch_float64(approx):
    x = (rng.standard_normal(4096) * 4).astype(np.float32)
    ref = F.gelu(t64(x), approximate=approx).numpy()
    np.testing.assert_allclose(oracle.gelu(x, approx), ref, rtol=1e-6, atol=1e-7)


def test_gelu_closed_forms():
    x = np.array([0.0, 30.0, -30.0, 1.0], np.float32)
    g = oracle.gelu(x, "none")
    assert g[0] == 0.0 and g[1] == 30.0 and abs(g[2]) < 1e-30
    # gelu(x) - gelu(-x) = x for the erf form (Phi(x) + Phi(-x) = 1)
    y = (rng.standard_normal(100) * 3).astype(np.float32)
    np.testing.assert_allclose(oracle.gelu(y) - oracle.gelu(-y), y, rtol=1e-5, atol=1e-6)
    # gelu(1) = 0.5 * (1 + erf(1/sqrt 2)) = Phi(1)
    assert abs(g[3] - 0.5 * (1 + math.erf(1 / math.sqrt(2)))) < 1e-7


def test_bias_gelu_matches_torch():
    x = rng.standard_normal((64, 96)).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    ref = F.gelu(t64(x) + t64(b), approximate="tanh").numpy()
    np.testing.assert_allclose(oracle.bias_gelu(x, b, "tanh"), ref, rtol=1e-6, atol=1e-7)


def test_layernorm_matches_torch_and_invariants():
    x = (rng.standard_normal((37, 768)) * 3 + 1).astype(np.float32)
    g = (1 + rng.standard_normal(768) * 0.02).astype(np.float32)
    b = (rng.standard_normal(768) * 0.02).astype(np.float32)
    ref = F.layer_norm(t64(x), (768,), t64(g), t64(b), 1e-5).numpy()
    np.testing.assert_allclose(oracle.layernorm(x, g, b), ref, rtol=1e-6, atol=1e-6)
    y = oracle.layernorm(x).astype(np.float64)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-6)
    var = x.astype(np.float64).var(-1)
    np.testing.assert_allclose((y ** 2).mean(-1), var / (var + 1e-5), rtol=1e-5)


def test_layernorm_eps_matters():
    x = np.full((1, 8), 3.0, np.float32)
    x[0, 0] = 3.001
    # tiny variance: the result depends on eps being added
    y = oracle.layernorm(x, eps=1e-5)
    ref = F.layer_norm(t64(x), (8,), eps=1e-5).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-7)


def test_softmax_matches_torch_and_invariants():
    x = rng.standard_normal((12, 7, 512)).astype(np.float32)
    ref = F.softmax(t64(x) * 0.125, -1).numpy()
    s = oracle.softmax(x, 0.125)
    np.testing.assert_allclose(s, ref, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(s.astype(np.float64).sum(-1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(oracle.softmax(x + 17.0), oracle.softmax(x), rtol=1e-5, atol=1e-9)
    m = np.full((2, 4), -np.inf, np.float32)
    m[0, :2] = [0.0, 0.0]
    out = oracle.softmax(m)
    np.testing.assert_allclose(out[0], [0.5, 0.5, 0, 0])
    assert np.isnan(out[1]).all()           # an all -inf row is NaN, as in torch


def test_matmul_matches_torch_and_closed_forms():
    a = rng.standard_normal((3, 17, 33)).astype(np.float32)
    b = rng.standard_normal((3, 33, 9)).astype(np.float32)
    np.testing.assert_allclose(oracle.matmul(a, b), (t64(a) @ t64(b)).numpy(), rtol=1e-6, atol=1e-6)
    eye = np.eye(33, dtype=np.float32)
    np.testing.assert_array_equal(oracle.matmul(a[0], eye), a[0])
    u, v = rng.standard_normal((5, 1)).astype(np.float32), rng.standard_normal((1, 6)).astype(np.float32)
    np.testing.assert_allclose(oracle.matmul(u, v), u.astype(np.float64) * v, rtol=1e-7)
    # brute force on a tiny case
    small_a, small_b = a[0, :2, :3], b[0, :3, :2]
    brute = [[sum(float(small_a[i, k]) * float(small_b[k, j]) for k in range(3)) for j in range(2)] for i in range(2)]
    np.testing.assert_allclose(oracle.matmul(small_a, small_b), brute, rtol=1e-6)


@pytest.mark.parametrize("act", ["none", "tanh", "erf"])
def test_linear_matches_torch(act):
    x = rng.standard_normal((16, 64)).astype(np.float32)
    w = (rng.standard_normal((48, 64)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(48) * 0.02).astype(np.float32)
    r = rng.standard_normal((16, 48)).astype(np.float32)
    y = F.linear(t64(x), t64(w), t64(b))
    if act != "none":
        y = F.gelu(y, approximate="tanh" if act == "tanh" else "none")
    y = y + t64(r)
    np.testing.assert_allclose(oracle.linear(x, w.T, b, r, act), y.numpy(), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("d,nh,T", [(64, 4, 16), (96, 3, 33)])
def test_block_matches_torch_float64(d, nh, T):
    torch.manual_seed(0)
    model = gpt2_init_(Block(d, nh, T), seed=3).double().eval()
    x = rng.standard_normal((T, d)).astype(np.float32)
    with torch.no_grad():
        ref = model(t64(x)).numpy()
    params = {k: v.float().numpy() for k, v in model.state_dict().items()}
    np.testing.assert_allclose(oracle.block(x, params, nh), ref, rtol=1e-5, atol=1e-6)


def test_block_is_causal():
    # the first P rows depend only on the first P inputs (used by the GPU tests)
    torch.manual_seed(0)
    model = gpt2_init_(Block(64, 4, 24), seed=2).eval()
    params = {k: v.numpy() for k, v in model.state_dict().items()}
    x = rng.standard_normal((24, 64)).astype(np.float32)
    full = oracle.block(x, params, 4)
    np.testing.assert_array_equal(oracle.block(x[:10], params, 4), full[:10])
    y = x.copy()
    y[15:] += 1.0
    np.testing.assert_array_equal(oracle.block(y, params, 4)[:15], full[:15])


def test_interpreter_matches_torch_on_an_imported_model():
    from kiln.frontend.fx_import import import_exported

    torch.manual_seed(0)
    model = Block(32, 2, 8).eval()
    x = torch.randn(8, 32)
    g = import_exported(torch.export.export(model, (x,)).run_decompositions())
    with torch.no_grad():
        ref = model.double()(x.double()).numpy()
    (out,) = interp.run(g, x.numpy())
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_interpreter_ops_brute_force():
    from kiln.ir import parse

    g = parse("""
    graph @f(%arg0: f32[2, 3]) -> (f32[2, 1], f32[3, 2], f32[2, 3]) {
      %0 = reduce_max %arg0 {dims = [1]} : f32[2, 1]
      %1 = transpose %arg0 {perm = [1, 0]} : f32[3, 2]
      %2 = const {value = 0.5} : f32[]
      %3 = maximum %arg0, %2 : f32[2, 3]
      return %0, %1, %3
    }""")
    x = np.array([[1.0, -2.0, 0.25], [0.0, 3.0, -1.0]], np.float32)
    mx, tr, clip = interp.run(g, x)
    assert mx.tolist() == [[1.0], [3.0]]
    assert tr.tolist() == [[1.0, 0.0], [-2.0, 3.0], [0.25, -1.0]]
    assert clip.tolist() == [[1.0, 0.5, 0.5], [0.5, 3.0, 0.5]]


def test_bf16_round_matches_torch_and_known_answers():
    # torch's float -> bfloat16 conversion (round to nearest, ties to even) is
    # the library routine; the oracle computes the rounding arithmetically
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(200_000) * 10.0 ** rng.integers(-44, 38, 200_000)).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oracle.bf16_round(x), want)
    one = np.float32(1.0)
    cases = {
        1 + 2.0 ** -8: 1.0,                  # tie -> even (1.0)
        1 + 3 * 2.0 ** -8: 1 + 2.0 ** -6,    # tie -> even (mantissa ...10)
        1 + 2.0 ** -8 + 2.0 ** -12: 1 + 2.0 ** -7,   # above the tie
        -(1 + 2.0 ** -7): -(1 + 2.0 ** -7),  # exact
        3.4e38: np.inf,                      # past the largest finite bf16
        2.0 ** -133: 2.0 ** -133,            # smallest subnormal
        2.0 ** -134: 0.0,                    # half of it: tie -> even (0)
    }
    got = oracle.bf16_round(np.array(list(cases), np.float32))
    np.testing.assert_array_equal(got, np.array(list(cases.values()), np.float32))
    special = oracle.bf16_round(np.array([np.nan, np.inf, -np.inf, -0.0], np.float32))
    assert np.isnan(special[0]) and special[1] == np.inf and special[2] == -np.inf
    assert special[3] == 0 and np.signbit(special[3])
    assert oracle.bf16_round(np.array([one], np.float32))[0] == one
