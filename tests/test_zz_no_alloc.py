"""kh_plan_run_noalloc: kh_plan_run with the split-K partials in the
library's own device array instead of a caller workspace (for callers that
cannot allocate device memory). Called through the C ABI (ctypes) and checked
bit for bit against kh_plan_run on the same plan and inputs."""

import ctypes

import pytest
import torch
import torch.nn.functional as F

import kiln
from kiln.hip import lib as kl


def _split_k_program(m, n, k, splitk):
    a, b, bias = torch.randn(m, k), torch.randn(k, n) * 0.05, torch.randn(n)
    fn = lambda a, b, bias: F.gelu(a @ b + bias, approximate="tanh")
    compiled = kiln.compile(fn, (a, b, bias), device="cuda", cuda_graphs=False,
                            gpu_matmul_config=lambda *_: {"tile": 2, "splitk": splitk})
    return compiled, (a, b, bias)


def _unbound_workspace_plan(compiled):
    """A second plan over the same launches, bound to the compiled graph's
    constants and arena but to no workspace."""
    exe = compiled._exe
    plan = kl.Plan([l.desc for l in exe.program.launches])
    plan.bind([t.data_ptr() for t in exe.constants], exe.arena.data_ptr(), None, 0)
    return plan


@pytest.mark.gpu
def test_noalloc_run_matches_kh_plan_run_on_consecutive_calls():
    lib = kl.load()
    # the second call is smaller than the first, so any partial it reads
    # that it did not write itself would hold the first call's values
    for m, n, k, splitk in ((128, 768, 3072, 6), (64, 256, 1024, 4)):
        compiled, xs = _split_k_program(m, n, k, splitk)
        plan = _unbound_workspace_plan(compiled)
        assert 0 < plan.workspace_bytes == splitk * m * n * 4 <= kl.NOALLOC_WORKSPACE_BYTES
        print(f"noalloc: M={m} N={n} K={k} split-K {splitk}", flush=True)
        expected = compiled(*xs)
        ins = [x.to("cuda").contiguous() for x in xs]
        out = torch.full((m, n), float("nan"), device="cuda")
        in_arr, out_arr = kl.pointer_array([t.data_ptr() for t in ins]), kl.pointer_array([out.data_ptr()])
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        kl.check(lib.kh_plan_run_noalloc(plan.handle, in_arr, len(ins), out_arr, 1, stream), "kh_plan_run_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, expected)


@pytest.mark.gpu
def test_unbound_workspace_is_refused_by_kh_plan_run():
    compiled, xs = _split_k_program(128, 768, 3072, 6)
    plan = _unbound_workspace_plan(compiled)
    ins = [x.to("cuda") for x in xs]
    out = torch.empty(128, 768, device="cuda")
    with pytest.raises(MemoryError, match="kh_plan_run_noalloc"):
        plan.run([t.data_ptr() for t in ins], [out.data_ptr()], torch.cuda.current_stream().cuda_stream)


def test_noalloc_rejects_plans_beyond_its_array():
    # 2048 x 3072 split 4: 96 MiB of partials > 16 MiB; refused before any launch

    import test_lowering

    _, prog = test_lowering.lowered(lambda a, b: a @ b, torch.randn(2048, 768), torch.randn(768, 3072))
    d = kl.LaunchDesc.from_buffer_copy(prog.launches[0].desc)
    d.cfg[1], d.cfg[2] = 2, 4
    plan = kl.Plan([d])
    assert plan.workspace_bytes == 4 * 2048 * 3072 * 4 > kl.NOALLOC_WORKSPACE_BYTES
    plan.bind([], None, None, 0)
    null = kl.pointer_array([None])
    rc = plan.lib.kh_plan_run_noalloc(plan.handle, null, 1, null, 1, None)
    assert rc == kl.ERR_CAPACITY
    assert b"16777216" in plan.lib.kh_last_error()


def _captured_noalloc(plan, ins, out):
    """kh_plan_run_noalloc recorded into a torch CUDA graph: a device
    allocation during the call would fail the capture."""
    lib = kl.load()
    in_arr, out_arr = kl.pointer_array([t.data_ptr() for t in ins]), kl.pointer_array([out.data_ptr()])
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            kl.check(lib.kh_plan_run_noalloc(plan.handle, in_arr, len(ins), out_arr, 1, stream),
                     "kh_plan_run_noalloc")
    torch.cuda.current_stream().wait_stream(side)
    return graph, (in_arr, out_arr)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["split-k", "decode-chain"])
def test_noalloc_run_captures_into_a_graph(case):
    # the promise of the entry point: it allocates nothing, so it can be
    # captured; each replay (with the program's own eager work between
    # replays) matches kh_plan_run bit for bit
    from models.transformer import Stack, gpt2_init_

    if case == "split-k":
        compiled, xs = _split_k_program(128, 768, 3072, 6)
        shape = (128, 768)
    else:
        torch.manual_seed(0)
        model = gpt2_init_(Stack(2, 128, 4, 1), seed=0).eval()
        xs = (torch.randn(1, 128),)
        compiled = kiln.compile(model, xs, device="cuda", cuda_graphs=False, gemv_chains=True)
        assert compiled.report.lowering["gemv_chains"]
        shape = (1, 128)
    print(f"noalloc capture: {case}", flush=True)
    plan = _unbound_workspace_plan(compiled)
    expected = compiled(*xs)
    ins = [x.to("cuda").contiguous() for x in xs]
    out = torch.full(shape, float("nan"), device="cuda")
    graph, keep = _captured_noalloc(plan, ins, out)
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
        _ = (ins[0] * 2.0).sum().item()   # eager work between replays
    assert plan.chain_timeouts() == 0
