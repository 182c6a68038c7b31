"""The bf16-input GEMM variant, host side: weight copies, lowering and the
library's descriptor checks (no GPU needed). Results are checked on the GPU in
tests/test_gpu_bf16.py."""

import numpy as np
import pytest
import torch

import oracle
from kiln.api import Options, build_passes
from kiln.frontend.fx_import import import_exported
from kiln.hip import autotune, bf16
from kiln.hip import lib as kl
from kiln.hip.lowering import lower_graph
from kiln.passes.manager import PassManager


def lowered(fn, *xs, precision="bf16"):
    module = fn if isinstance(fn, torch.nn.Module) else type("F", (torch.nn.Module,), {
        "forward": lambda self, *a: fn(*a)})()
    g = import_exported(torch.export.export(module.eval(), xs).run_decompositions())
    PassManager(build_passes(Options())).run(g)
    return g, lower_graph(g, precision=precision)


def test_bf16_bits_match_the_oracle_rounding():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100_000) * 10.0 ** rng.integers(-44, 38, 100_000)).astype(np.float32)
    x[:4] = [np.nan, np.inf, -np.inf, -0.0]
    bits = bf16.bf16_bits(x)
    as_f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    want = oracle.bf16_round(x)
    assert np.isnan(as_f32[0])
    np.testing.assert_array_equal(as_f32[1:], want[1:])


def test_weight_copy_is_n_by_padded_k():
    w = np.arange(5 * 11, dtype=np.float32).reshape(5, 11) / 7  # [K=5, N=11] row-major
    copy = bf16.weight_copy(w, 0, (0, 11, 1), 1, 5, 11)
    assert copy.shape == (1, 11, 8) and copy.dtype == np.uint16
    vals = (copy.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(vals[0, :, :5], oracle.bf16_round(w.T))
    assert not vals[0, :, 5:].any()
    # a strided view (every other column, offset 1) of a batched constant
    w3 = np.random.default_rng(0).standard_normal((2, 4, 10)).astype(np.float32)
    copy3 = bf16.weight_copy(w3, 1, (40, 10, 2), 2, 4, 4)
    vals3 = (copy3.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(vals3[:, :, :4], oracle.bf16_round(w3[:, :, 1:9:2].transpose(0, 2, 1)))


def test_linear_lowers_to_the_bf16_gemm_with_a_weight_copy():
    lin = torch.nn.Linear(61, 133)
    _, prog = lowered(lin, torch.randn(77, 61))
    (launch,) = prog.launches
    d = launch.desc
    assert launch.family == kl.FAM_GEMM and d.cfg[3] == kl.PREC_BF16
    assert autotune.PRECISION[d.cfg[1]] == "bf16" and "bf16" in launch.summary
    b = d.refs[1]
    name = prog.consts[b.index]
    assert b.base == kl.BASE_CONST and name in prog.derived
    assert (b.offset, b.strides[0], b.strides[1], b.strides[2]) == (0, 0, 1, 64)   # K' = 64
    src, offset, strides, batch, k, n = prog.derived[name]
    assert (batch, k, n) == (1, 61, 133) and strides[2] == 1 and strides[1] == 133
    # the fp32 original is read only through the copy: it is not uploaded
    assert src not in prog.consts


def test_bf16_decode_and_activation_products():
    # M = 1 with a constant weight and K a multiple of 8 runs on the GEMV
    # family over the bf16 [N][K] copy; K = 61 (partial 16-byte chunks) on the
    # bf16 GEMM tiles
    _, prog = lowered(torch.nn.Linear(768, 3072), torch.randn(1, 768))
    d = prog.launches[0].desc
    assert prog.launches[0].family == kl.FAM_GEMV and d.cfg[3] == kl.PREC_BF16
    assert (d.refs[1].base, d.refs[1].strides[1], d.refs[1].strides[2]) == (kl.BASE_CONST, 1, 768)
    kl.Plan([d])
    _, prog = lowered(torch.nn.Linear(61, 30), torch.randn(1, 61))
    assert prog.launches[0].family == kl.FAM_GEMM and prog.launches[0].desc.cfg[3] == kl.PREC_BF16
    # a product of two activations has no constant to copy: it stays fp32
    _, prog = lowered(lambda a, b: a @ b, torch.randn(64, 32), torch.randn(32, 48))
    d = prog.launches[0].desc
    assert d.cfg[3] == kl.PREC_FP32 and autotune.PRECISION[d.cfg[1]] == "fp32" and not prog.derived


def test_library_checks_bf16_descriptors():
    _, prog = lowered(torch.nn.Linear(64, 96), torch.randn(32, 64))
    good = kl.LaunchDesc.from_buffer_copy(prog.launches[0].desc)
    kl.Plan([good])
    bad = kl.LaunchDesc.from_buffer_copy(good)
    bad.cfg[1] = 0          # an fp32 configuration
    with pytest.raises(ValueError, match="another precision"):
        kl.Plan([bad])
    bad = kl.LaunchDesc.from_buffer_copy(good)
    bad.refs[1].strides[2] = 60   # K' not a multiple of 8
    with pytest.raises(ValueError, match="bf16 B operand"):
        kl.Plan([bad])


def test_bf16_defaults_and_candidates_are_bf16_tiles():
    for m, n, k in [(2048, 3072, 768), (128, 768, 3072), (1, 2304, 768)]:
        d = autotune.default_config_for(1, m, n, k, cus=256, precision="bf16")
        assert autotune.PRECISION[d["tile"]] == "bf16"
        assert all(autotune.PRECISION[c["tile"]] == "bf16"
                   for c in autotune.candidates(1, m, n, k, cus=256, precision="bf16"))


def test_three_pass_weight_copy_layout_and_values():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((2, 13, 11)).astype(np.float32)          # [batch, K, N], K not a multiple of 8
    w[0, 0, 0], w[1, 2, 3] = np.inf, np.nan
    out = bf16.weight_copy_x3(w, 0, (13 * 11, 11, 1), 2, 13, 11)
    kp = bf16.padded_k(13)
    assert out.shape == (2, 11, 2 * kp) and out.dtype == np.uint16
    np.testing.assert_array_equal(out[:, :, :kp], bf16.weight_copy(w, 0, (13 * 11, 11, 1), 2, 13, 11))
    assert not out[:, :, 13:kp].any() and not out[:, :, kp + 13:].any()
    hi = bf16.bf16_value(out[:, :, :13]).transpose(0, 2, 1)
    lo = bf16.bf16_value(out[:, :, kp:kp + 13]).transpose(0, 2, 1)
    # the hi + lo split is checked against the C oracle's rounding
    finite = np.isfinite(w)
    np.testing.assert_array_equal(hi[finite], oracle.bf16_round(w)[finite])
    np.testing.assert_array_equal(lo[finite], oracle.bf16_round((w - hi).astype(np.float32))[finite])
    assert np.all(np.abs((hi[finite] + lo[finite]) - w[finite]) <= 2.0 ** -16 * np.abs(w[finite]))
    assert hi[0, 0, 0] == np.inf and lo[0, 0, 0] == 0.0 and np.isnan(hi[1, 2, 3]) and lo[1, 2, 3] == 0.0


def test_allow_tf32_lowers_to_the_three_pass_gemm():
    lin = torch.nn.Linear(64, 40).eval()
    g = import_exported(torch.export.export(lin, (torch.randn(32, 64),)).run_decompositions())
    PassManager(build_passes(Options(device="cuda", allow_tf32=True))).run(g)
    prog = lower_graph(g, precision="bf16x3")
    (l,) = prog.launches
    assert l.desc.cfg[3] == kl.PREC_BF16X3 and autotune.PRECISION[l.desc.cfg[1]] == "bf16x3"
    (name,) = [n for n in prog.derived if "@bf16x3:" in n]
    assert list(l.desc.refs[1].strides)[:3] == [0, 1, 2 * bf16.padded_k(64)]
    kl.Plan([l.desc for l in prog.launches])
