"""The HIP backend's host side on the CPU: the C-ABI library loads and exports
every entry point of include/kiln_hip.h, descriptors are validated by the
library (kh_plan_create runs without a GPU: it only prepares kernel
arguments), and the lowering picks the intended kernel families."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kiln.api import Options, build_passes, compile_graph
from kiln.frontend.fx_import import import_exported
from kiln.hip import autotune, lib as kl
from kiln.hip.lowering import lower_graph
from kiln.ir import parse
from kiln.passes.manager import PassManager
from models.transformer import Block, Stack

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "kiln_hip.h")
PKG_ROOT = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kiln-compiler_amd")


def lowered(fn, *xs, fuse_attention=False, **opts):
    module = fn if isinstance(fn, torch.nn.Module) else type("F", (torch.nn.Module,), {
        "forward": lambda self, *a: fn(*a)})()
    g = import_exported(torch.export.export(module.eval(), xs).run_decompositions())
    passes = build_passes(Options(**opts))
    if fuse_attention:
        from kiln.hip.attention import FuseAttention

        passes.insert(len(passes) - 1, FuseAttention())
    PassManager(passes).run(g)
    return g, lower_graph(g)


def test_library_exports_every_header_symbol():
    lib = kl.load()
    declared = set(re.findall(r"^\s*(?:int|const char \*)\s*(kh_\w+)\s*\(", open(HEADER).read(), re.M))
    assert declared == set(kl.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.kh_version() == kl.ABI_VERSION


def test_library_build_id_is_the_tree_digest():
    # kh_build_id (part of the stored-plan key) is the digest of the sources
    # the library was built from: a library built from other sources gives
    # other plan keys
    import importlib.util

    spec = importlib.util.spec_from_file_location("kiln_hip_build", os.path.join(PKG_ROOT, "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    assert kl.build_id() == build.source_digest()
    assert len(kl.build_id()) == 32


def test_struct_sizes_match_the_library():
    sizes = (ctypes.c_size_t * 4)()
    kl.load().kh_abi_sizes(sizes)
    assert tuple(sizes) == (ctypes.sizeof(kl.LaunchDesc), ctypes.sizeof(kl.Ref), ctypes.sizeof(kl.Insn),
                            ctypes.sizeof(kl.PassDesc))


def test_gemm_config_table_matches_the_tuner():
    cfgs = kl.gemm_configs()
    assert len(cfgs) == len(autotune.TILES)
    for i, c in enumerate(cfgs):
        assert tuple(c[:7]) == autotune.TILES[i]


def test_block_lowers_to_the_expected_families():
    g, prog = lowered(Block(768, 12, 128), torch.randn(128, 768))
    fams = [kl.FAMILY_NAMES[l.family] for l in prog.launches]
    # both LayerNorms run as the prologue of the small-M GEMM that reads them
    # (qkv, MLP up): no row launch of their own
    assert fams == ["gemm", "elementwise", "gemm", "row", "gemm", "elementwise", "gemm", "gemm", "gemm"]
    variants = [l.desc.variant for l in prog.launches if l.family == kl.FAM_ROW]
    assert variants == [kl.ROW_SOFTMAX]
    assert [i for i, l in enumerate(prog.launches) if "prologue: layernorm" in l.summary] == [0, 7]
    plan = kl.Plan([l.desc for l in prog.launches])
    assert plan.n_launches == 9


def test_block_attention_becomes_one_launch():
    T = 256
    g, prog = lowered(Block(768, 12, T), torch.randn(T, 768), fuse_attention=True)
    fams = [kl.FAMILY_NAMES[l.family] for l in prog.launches]
    assert fams == ["row", "gemm", "attention", "gemm", "row", "gemm", "gemm"]
    a = prog.launches[2].desc
    assert (a.cfg[0], a.cfg[1], a.fparams[0]) == (kl.ATTN_MASK_CAUSAL, kl.ATTN_SCALE_MUL, 0.125)
    assert tuple(a.gemm) == (12, T, T, 64) and a.n_refs == 4
    # q, k, v are column blocks of the qkv buffer [T, 2304]; the output is the
    # head-merged [T, 768] layout the projection reads
    strides = [tuple(a.refs[j].strides[:3]) for j in range(4)]
    assert strides == [(64, 2304, 1)] * 3 + [(64, 768, 1)]
    assert [a.refs[j].offset - a.refs[0].offset for j in range(3)] == [0, 768, 1536]
    # no [12, T, T] buffer is planned: the peak is now the MLP (residual,
    # ln2 output and fc output live together), (768 + 768 + 3072) T floats
    assert g.attrs["arena_bytes"] == 4 * 4608 * T
    kl.Plan([l.desc for l in prog.launches])


class _Attn(torch.nn.Module):
    def __init__(self, mask=None, divide=False):
        super().__init__()
        self.divide = divide
        if mask is not None:
            self.register_buffer("mask", mask)
        else:
            self.mask = None

    def forward(self, q, k, v):
        s = q @ k.transpose(-2, -1)
        s = s / 8.0 if self.divide else s * 0.125
        if self.mask is not None:
            s = s + self.mask
        return F.softmax(s, dim=-1) @ v


@pytest.mark.parametrize("d, mask, divide, want", [
    (64, None, False, (kl.ATTN_MASK_NONE, kl.ATTN_SCALE_MUL, 4)),
    (32, torch.randn(40, 40), True, (kl.ATTN_MASK_ADD, kl.ATTN_SCALE_DIV, 5)),
    (64, torch.full((40, 40), float("-inf")).triu(1), False, (kl.ATTN_MASK_CAUSAL, kl.ATTN_SCALE_MUL, 4)),
    (64, torch.full((40, 40), float("-inf")).triu(2), False, (kl.ATTN_MASK_ADD, kl.ATTN_SCALE_MUL, 5)),
])
def test_attention_modes(d, mask, divide, want):
    xs = [torch.randn(3, 40, d) for _ in range(3)]
    _, prog = lowered(_Attn(mask, divide), *xs, fuse_attention=True)
    attn = [l.desc for l in prog.launches if l.family == kl.FAM_ATTN]
    assert len(attn) == 1
    assert (attn[0].cfg[0], attn[0].cfg[1], attn[0].n_refs) == want
    kl.Plan([l.desc for l in prog.launches])


def test_attention_needs_a_supported_head_dim():
    xs = [torch.randn(2, 24, 16) for _ in range(3)]
    _, prog = lowered(_Attn(), *xs, fuse_attention=True)
    assert kl.FAM_ATTN not in [l.family for l in prog.launches]


def test_attention_descriptor_checks():
    xs = [torch.randn(2, 24, 64) for _ in range(3)]
    _, prog = lowered(_Attn(), *xs, fuse_attention=True)
    d = next(l.desc for l in prog.launches if l.family == kl.FAM_ATTN)
    bad = kl.LaunchDesc.from_buffer_copy(d)
    bad.refs[1].strides[2] = 2
    with pytest.raises(NotImplementedError, match="unit head-dim stride"):
        kl.Plan([bad])
    bad = kl.LaunchDesc.from_buffer_copy(d)
    bad.cfg[0] = 7
    with pytest.raises(ValueError, match="mask or scale mode"):
        kl.Plan([bad])


def test_decode_uses_the_gemv_family():
    _, prog = lowered(torch.nn.Linear(768, 3072), torch.randn(1, 768))
    assert [l.family for l in prog.launches] == [kl.FAM_GEMV]


def test_gemv_weights_are_k_contiguous_copies():
    # a constant GEMV weight is read as a derived [N][K] copy (the nn.Linear
    # layout) holding exactly the frozen W^T's values; K not a multiple of 4
    # keeps the [K][N] constant
    from kiln.hip.runtime import host_constant, nk_copy

    lin = torch.nn.Linear(768, 300)
    g, prog = lowered(lin, torch.randn(1, 768))
    (name,) = [n for n in prog.derived if "@nk:" in n]
    d = prog.launches[0].desc
    assert (d.refs[1].strides[1], d.refs[1].strides[2]) == (1, 768)
    src, offset, strides, batch, k, n = prog.derived[name]
    copy = nk_copy(g.constants[src], offset, strides, batch, k, n)
    assert copy.shape == (1, 300, 768) and copy.flags.c_contiguous
    np.testing.assert_array_equal(copy[0], lin.weight.detach().numpy())
    assert host_constant(prog, g.constants, name).shape == (1, 300, 768)
    # the frozen W^T itself is read only through the copy: it gets no slot
    assert name in prog.consts and src not in prog.consts
    _, prog = lowered(torch.nn.Linear(37, 30), torch.randn(1, 37))
    assert not prog.derived


def test_long_rows_are_chunked_and_short_rows_fast():
    _, prog = lowered(torch.nn.LayerNorm(10000), torch.randn(2, 10000))
    assert "(chunked)" in prog.launches[0].summary
    _, prog = lowered(torch.nn.LayerNorm(768), torch.randn(4, 768))
    assert prog.launches[0].desc.variant == kl.ROW_LAYERNORM
    _, prog = lowered(lambda x: F.softmax(x * 0.125, -1), torch.randn(2, 8, 64))
    d = prog.launches[0].desc
    assert d.variant == kl.ROW_SOFTMAX and d.cfg[4] == 1 and d.fparams[0] == 0.125


def test_column_reductions_use_the_reduce_family():
    _, prog = lowered(lambda x: x.sum(0, keepdim=True) * 2.0, torch.randn(6, 10))
    assert kl.FAM_RED in [l.family for l in prog.launches]


def test_bias_gelu_is_one_elementwise_launch_with_vector_operands():
    b = torch.randn(3072)
    _, prog = lowered(lambda t: F.gelu(t + b, approximate="tanh"), torch.randn(64, 3072))
    (launch,) = prog.launches
    assert launch.family == kl.FAM_EW
    ops = [kl.OPCODES[launch.desc.insns[i].op] for i in range(launch.desc.n_insns)]
    assert ops == ["load", "load", "add", "gelu_tanh", "store"]
    bias = launch.desc.refs[1] if launch.desc.refs[0].strides[0] else launch.desc.refs[0]
    assert list(bias.strides[:2]) == [0, 1]


def test_layernorm_prologue_only_up_to_its_row_limit():
    # past LN_PROLOGUE_MAX_ROWS rows the LayerNorm keeps its own launch (the
    # prologue's row statistics would cost the product more than the launch)
    from kiln.hip import lowering

    lim = lowering.LN_PROLOGUE_MAX_ROWS
    for rows, fused in ((lim, True), (lim + 32, False)):
        cfg = lambda *_: {"tile": 66, "splitk": 1}
        g = import_exported(torch.export.export(_ln_linear().eval(), (torch.randn(rows, 64),)).run_decompositions())
        PassManager(build_passes(Options())).run(g)
        prog = lower_graph(g, matmul_config=cfg)
        assert any("prologue: layernorm" in l.summary for l in prog.launches) == fused


@pytest.mark.parametrize("prec, b_bytes", [("fp32", 4), ("bf16", 2), ("bf16x3", 4)])
def test_matmul_launch_bytes_count_the_weight_copy_read(prec, b_bytes):
    # algorithmic bytes of a Linear: A, the bias and the output in fp32, the
    # weights as the copy the kernel reads (bf16: 2 bytes a weight; the
    # three-pass copy holds two bf16 per weight)
    m, k, n = 64, 96, 80
    g = import_exported(torch.export.export(torch.nn.Linear(k, n).eval(), (torch.randn(m, k),)).run_decompositions())
    PassManager(build_passes(Options())).run(g)
    prog = lower_graph(g, precision=prec, matmul_config=lambda *_: {"tile": autotune.default_config_for(
        1, m, n, k, precision=prec)["tile"], "splitk": 1})
    (launch,) = prog.launches
    assert launch.bytes == 4 * (m * k + n + m * n) + b_bytes * k * n


def test_stack_decode_plan():
    _, prog = lowered(Stack(12, 768, 12, 1), torch.randn(1, 768))
    # ln_1 and ln_2 of every layer run as the prologue of the qkv / fc GEMV;
    # the final LayerNorm feeds the output and stays a row kernel
    assert len(prog.launches) == 12 * 7 + 1
    assert sum("prologue: layernorm" in l.summary for l in prog.launches) == 24
    assert kl.FAMILY_NAMES[prog.launches[-1].family] == "row"
    kl.Plan([l.desc for l in prog.launches])


def test_decode_attention_runs_as_the_projection_prologue():
    _, prog = lowered(Block(768, 12, 1), torch.randn(1, 768), fuse_attention=True)
    # ln_1 -> qkv, attention -> c_proj, ln_2 -> fc, proj: four GEMVs
    assert [kl.FAMILY_NAMES[l.family] for l in prog.launches] == ["gemv"] * 4
    assert "prologue: attention" in prog.launches[1].summary
    # (cfg[7] counts the keys: the summary does not read it as bf16 storage)
    assert not any("bf16" in l.summary for l in prog.launches)
    d = prog.launches[1].desc
    assert (d.cfg[0], d.cfg[4], d.cfg[7]) == (64, kl.GEMV_PRO_ATTN, 1)
    kl.Plan([l.desc for l in prog.launches])
    for field, value in ((7, 65), (0, 48), (5, 1)):
        bad = kl.LaunchDesc.from_buffer_copy(d)
        bad.cfg[field] = value
        with pytest.raises(ValueError, match="attention prologue"):
            kl.Plan([bad])


def _ln_linear(affine=True, bias=True):
    ln = torch.nn.LayerNorm(64, elementwise_affine=affine)
    lin = torch.nn.Linear(64, 48, bias=bias)
    return torch.nn.Sequential(ln, lin).eval()


@pytest.mark.parametrize("affine", [True, False])
def test_layernorm_feeding_a_gemv_becomes_its_prologue(affine):
    _, prog = lowered(_ln_linear(affine), torch.randn(1, 64))
    assert [kl.FAMILY_NAMES[l.family] for l in prog.launches] == ["gemv"]
    d = prog.launches[0].desc
    assert d.cfg[4] == 1 and "prologue: layernorm" in prog.launches[0].summary
    if affine:
        assert 2 <= d.cfg[5] < d.n_refs and 2 <= d.cfg[6] < d.n_refs and d.cfg[5] != d.cfg[6]
    else:
        assert d.cfg[5] == -1 and d.cfg[6] == -1
    assert list(d.fparams)[:3] == pytest.approx([1 / 64, 1 / 64, 1e-5])
    kl.Plan([l.desc for l in prog.launches])


def test_layernorm_is_not_fused_when_its_output_has_other_users():
    ln, lin = torch.nn.LayerNorm(64), torch.nn.Linear(64, 48)
    _, prog = lowered(lambda x: (lin(ln(x)), ln(x) * 2.0), torch.randn(1, 64))
    assert "row" in [kl.FAMILY_NAMES[l.family] for l in prog.launches]
    assert not any(l.desc.cfg[4] for l in prog.launches if l.family == kl.FAM_GEMV)


@pytest.mark.parametrize("affine", [True, False])
def test_layernorm_feeding_a_small_m_gemm_becomes_its_prologue(affine):
    # a few rows: the product runs on an fp32 small-M configuration; A is the
    # LayerNorm's input, gamma is folded into the [N][K] weight copy, whose
    # column sums (ref cfg[5]) and beta . W (ref cfg[6]) are per-column
    # constants (strides 0 over M)
    _, prog = lowered(_ln_linear(affine), torch.randn(40, 64))
    assert [kl.FAMILY_NAMES[l.family] for l in prog.launches] == ["gemm"]
    launch = prog.launches[0]
    d = launch.desc
    assert d.cfg[1] in autotune.SMALL_M and d.cfg[4] == 1 and 2 <= d.cfg[5] < d.n_refs
    assert "prologue: layernorm" in launch.summary and d.refs[0].base == kl.BASE_INPUT
    assert list(d.fparams)[:3] == pytest.approx([1 / 64, 1 / 64, 1e-5])
    assert list(d.refs[d.cfg[5]].strides[:3]) == [0, 0, 1]
    names = [prog.consts[d.refs[j].index] for j in (1, d.cfg[5], d.cfg[6]) if j >= 0]
    assert "@lng:" in names[1]
    if affine:
        assert 2 <= d.cfg[6] < d.n_refs and list(d.refs[d.cfg[6]].strides[:3]) == [0, 0, 1]
        assert "@nkg:" in names[0] and "@lnc:" in names[2]
    else:
        assert d.cfg[6] == -1 and "@nk:" in names[0]
    kl.Plan([l.desc for l in prog.launches])


def test_layernorm_prologue_reads_merged_rows_through_a_reshape():
    # [3, 20, 64] -> LayerNorm -> reshape [60, 64] -> Linear: the product's A
    # is the caller's input itself, rows 64 elements apart
    _, prog = lowered(_ln_linear(), torch.randn(3, 20, 64))
    launch = prog.launches[0]
    assert kl.FAMILY_NAMES[launch.family] == "gemm" and "prologue: layernorm" in launch.summary
    a = launch.desc.refs[0]
    assert a.base == kl.BASE_INPUT and list(a.strides[:3]) == [0, 64, 1] and list(launch.desc.gemm)[:4] == [1, 60, 48, 64]
    assert not any("layernorm rows" in l.summary for l in prog.launches)


def test_folded_layernorm_plan_round_trips_through_the_store(tmp_path, monkeypatch):
    from kiln.hip import plans

    monkeypatch.setenv("KILN_CACHE_DIR", str(tmp_path))
    g, prog = lowered(_ln_linear(), torch.randn(40, 64))
    key = plans.plan_key(str(g), "fp32", "default", kl.device_info())
    plans.save(key, prog, [])
    back, _ = plans.load(key)
    assert back.derived == prog.derived and any("@lng:" in n for n in back.derived)
    assert bytes(back.launches[0].desc) == bytes(prog.launches[0].desc)


def test_folded_layernorm_constants():
    # the scaled weight copy is W^T row n times gamma; the column constants
    # are beta . W and the scaled copy's row sums (float64 sums)
    from kiln.hip.runtime import host_constant

    torch.manual_seed(3)
    model = _ln_linear()
    with torch.no_grad():
        model[0].weight.copy_(1 + 0.1 * torch.randn(64))
        model[0].bias.copy_(0.1 * torch.randn(64))
    g, prog = lowered(model, torch.randn(40, 64))
    d = prog.launches[0].desc
    w = model[1].weight.detach().numpy().astype(np.float64)      # [N, K]
    gam, bet = model[0].weight.detach().numpy(), model[0].bias.detach().numpy()
    scaled = host_constant(prog, g.constants, prog.consts[d.refs[1].index])
    np.testing.assert_array_equal(scaled[0], (w.astype(np.float32) * gam[None, :]).astype(np.float32))
    col = host_constant(prog, g.constants, prog.consts[d.refs[d.cfg[6]].index])
    np.testing.assert_allclose(col.reshape(-1), w @ bet.astype(np.float64), rtol=1e-6, atol=1e-7)
    sums = host_constant(prog, g.constants, prog.consts[d.refs[d.cfg[5]].index])
    np.testing.assert_allclose(sums.reshape(-1), scaled[0].astype(np.float64).sum(-1), rtol=1e-6, atol=1e-7)


def test_layernorm_stays_a_row_kernel_before_other_gemms():
    # more rows than the small-M kernel takes: the LayerNorm keeps its launch
    _, prog = lowered(_ln_linear(), torch.randn(1100, 64))
    assert [kl.FAMILY_NAMES[l.family] for l in prog.launches] == ["row", "gemm"]
    assert prog.launches[1].desc.cfg[4] == 0


@pytest.mark.parametrize("mutate, err", [
    (lambda d: setattr(d.insns[0], "op", 99), ValueError),
    (lambda d: setattr(d.insns[0], "dst", 40), ValueError),
    (lambda d: setattr(d, "family", 42), ValueError),
    (lambda d: setattr(d, "n_refs", 13), ValueError),
    (lambda d: d.cfg.__setitem__(1, 77), ValueError),
])
def test_library_rejects_bad_descriptors(mutate, err):
    _, prog = lowered(lambda a, b: a @ b + 1.0, torch.randn(8, 16), torch.randn(16, 4))
    d = kl.LaunchDesc.from_buffer_copy(prog.launches[0].desc)
    mutate(d)
    with pytest.raises(err):
        kl.Plan([d])


def test_unknown_precision_is_not_implemented():
    _, prog = lowered(lambda a, b: a @ b, torch.randn(8, 16), torch.randn(16, 4))
    d = kl.LaunchDesc.from_buffer_copy(prog.launches[0].desc)
    d.cfg[3] = 7
    with pytest.raises(NotImplementedError):
        kl.Plan([d])


def test_split_k_workspace_is_reported():
    _, prog = lowered(lambda a, b: a @ b, torch.randn(128, 3072), torch.randn(3072, 768))
    d = kl.LaunchDesc.from_buffer_copy(prog.launches[0].desc)
    d.cfg[1], d.cfg[2] = 2, 4          # 64x64 tiles, split-K 4
    plan = kl.Plan([d])
    # dense fp32 partials [split][batch][M][N]; no counters
    assert plan.workspace_bytes == 4 * 128 * 768 * 4


def test_plan_listing_is_stable():
    g = parse(open(os.path.join(os.path.dirname(__file__), "lit", "fusion.kir")).read())
    PassManager(build_passes(Options())).run(g)
    a, b = lower_graph(g), lower_graph(g)
    assert a.source == b.source and a.digest() == b.digest()


def test_default_tiles_fill_the_gpu():
    cfg = autotune.default_config_for(1, 2048, 3072, 768, cus=256)
    bm, bn = autotune.TILES[cfg["tile"]][:2]
    assert (2048 // bm) * (3072 // bn) * cfg["splitk"] >= 256
    small = autotune.default_config_for(1, 128, 768, 768, cus=256)
    bm, bn = autotune.TILES[small["tile"]][:2]
    assert -(-128 // bm) * -(-768 // bn) * small["splitk"] >= 64


def test_candidates_fit_the_problem():
    for m, n, k in [(128, 3072, 768), (7, 13, 5)]:
        for c in autotune.candidates(1, m, n, k, cus=256):
            bm, bn = autotune.TILES[c["tile"]][:2]
            assert bm <= max(16, 2 * m) and bn <= max(16, 2 * n)
    # M = 1 runs on the GEMV family: its candidates are workgroup variants
    gemv = autotune.candidates(1, 1, 768, 768, cus=256)
    assert {c["tile"] for c in gemv} == set(range(6)) and autotune.default_config_for(1, 1, 768, 768) in gemv


def test_options_and_errors():
    g = parse("graph @f(%arg0: f32[2]) -> (f32[2]) {\n %0 = exp %arg0 : f32[2]\n return %0\n}")
    with pytest.raises(ValueError):
        compile_graph(g, Options(device="tpu"))
    with pytest.raises(NotImplementedError):
        compile_graph(g, Options(device="cpu"))
    import kiln

    with pytest.raises(TypeError):
        kiln.compile(torch.nn.Linear(2, 2), (torch.randn(1, 2),), not_an_option=1)


def test_memory_check_gives_a_clear_error(monkeypatch):
    from kiln.hip.runtime import check_memory

    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda dev=None: (10 * 2**20, 32 * 2**30))
    with pytest.raises(MemoryError, match="only 10.0 MiB"):
        check_memory(torch.device("cuda"), 64 * 2**20, "the arena")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(kl, "_lib", None)
    monkeypatch.setenv("KILN_HIP_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="not built"):
        kl.load()


def test_autotune_cache_is_ignored_when_corrupt(tmp_path):
    autotune.cache_path().parent.mkdir(parents=True, exist_ok=True)
    autotune.cache_path().write_text("{not json")
    assert autotune.GPUAutotuner()._cache == {}


def test_shipped_tuning_table_is_consistent():
    table = autotune.shipped_configs()
    for key, entry in table.items():
        arch, cus, precision, shape = key.split("|")
        b, m, n, k = map(int, shape.split("x"))
        tile = entry["config"]["tile"]
        if precision.endswith("+a16"):      # timed reading a bf16 (bf16x3: pair-stored) A operand
            precision = precision[:-len("+a16")]
            assert precision in ("bf16", "bf16x3") and m > 1
        if m == 1 and precision == "fp32":
            assert 0 <= tile <= 5          # GEMV workgroup variants
        else:
            assert autotune.PRECISION[tile] == precision and (m == 1 or autotune.fits(tile, m, n, k))
        assert arch.startswith("gfx950") and int(cus) > 0


def test_tuner_never_times_a_spilling_configuration():
    for shape in ((1, 2048, 3072, 768), (1, 128, 768, 3072), (1, 300, 452, 96)):
        assert not any(c["tile"] in autotune.SPILLING for c in autotune.candidates(*shape, cus=256))
        assert autotune.default_config_for(*shape, cus=256)["tile"] not in autotune.SPILLING


def test_plans_round_trip_through_the_store(tmp_path, monkeypatch):
    # a stored plan reloads to byte-identical descriptors, the same constant
    # slots, derived-constant recipes and listing; a different key misses
    from kiln.hip import plans

    monkeypatch.setenv("KILN_CACHE_DIR", str(tmp_path))
    lin = torch.nn.Sequential(torch.nn.LayerNorm(768), torch.nn.Linear(768, 300), torch.nn.GELU())
    g, prog = lowered(lin, torch.randn(1, 768))
    assert prog.derived
    key = plans.plan_key(str(g), "fp32", "default", kl.device_info())
    listing = plans.save(key, prog, [])
    assert listing.read_text() == prog.source
    back, log = plans.load(key)
    assert log == [] and back.consts == prog.consts and back.derived == prog.derived
    assert [bytes(l.desc) for l in back.launches] == [bytes(l.desc) for l in prog.launches]
    assert back.source == prog.source and back.precision == prog.precision
    assert plans.load(plans.plan_key(str(g), "bf16", "default", kl.device_info())) is None
    # a damaged file is ignored, not trusted
    (tmp_path / "hip" / "plans" / f"{key}.json").write_text("{broken")
    assert plans.load(key) is None
