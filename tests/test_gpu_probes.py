"""The library's measurement probes (kh_probe_attn_timeline, kh_probe_mfma_valu).

The timeline probe runs the attention kernel itself, so its output is checked
like any attention output (float64 reference, fp32 tolerance); its records are
checked against what the launch must have done: every workgroup's key blocks
add up to its causal range, timestamps are ordered, clocks are plausible.
"""

import ctypes

import numpy as np
import pytest
import torch

from kiln.hip import lib as kl
from test_gpu import ATOL, RTOL

pytestmark = pytest.mark.gpu


def _causal_reference(q, k, v, scale):
    qd, kd, vd = (t.double().cpu() for t in (q, k, v))
    s = qd @ kd.transpose(1, 2) * scale
    T = s.shape[-1]
    s = s + torch.triu(torch.full((T, T), float("-inf"), dtype=torch.float64), 1)
    return torch.softmax(s, -1) @ vd


@pytest.mark.parametrize("waves", [4, 8])
def test_attention_timeline_runs_the_kernel_and_records_every_wave(waves):
    lib = kl.load()
    heads, T, DH = 2, 300, 64
    torch.manual_seed(3)
    qkv = torch.randn(T, 3 * heads * DH, device="cuda")
    out = torch.full((T, heads * DH), float("nan"), device="cuda")
    W = heads * DH
    q, k, v = qkv[:, :W], qkv[:, W:2 * W], qkv[:, 2 * W:]
    nq = (T + 31) // 32
    rec = torch.zeros(heads * nq * waves * 8, dtype=torch.int64, device="cuda")
    st = (ctypes.c_int64 * 8)(DH, 3 * W, DH, 3 * W, DH, 3 * W, DH, W)
    stream = torch.cuda.current_stream().cuda_stream
    kl.check(lib.kh_probe_attn_timeline(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), heads, T, T, st,
                                        waves, 0.125, rec.data_ptr(), stream), "kh_probe_attn_timeline")
    torch.cuda.synchronize()
    split = lambda t: t.reshape(T, heads, DH).permute(1, 0, 2)
    ref = _causal_reference(split(q), split(k), split(v), 0.125)
    got = split(out).double().cpu()
    assert torch.allclose(got, ref, rtol=RTOL, atol=ATOL), float((got - ref).abs().max())

    r = rec.cpu().numpy().reshape(heads * nq, waves, 8).view(np.uint64)
    for g in range(heads * nq):
        qb = nq - 1 - g // heads                      # longest-first order
        nkb = (min(T, 32 * qb + 32) + 31) // 32       # causal: key blocks up to the diagonal
        assert int(r[g, :, 7].sum()) == nkb
        assert np.all(r[g, :, 0] <= r[g, :, 1]) and np.all(r[g, :, 1] <= r[g, :, 2])
        assert np.all(r[g, :, 3] < r[g, :, 4])
    ghz = (r[:, :, 4] - r[:, :, 3]).astype(np.float64) / ((r[:, :, 2] - r[:, :, 0]).astype(np.float64) * 10.0)
    assert 0.5 < float(np.median(ghz)) < 3.5


def test_mfma_probe_measures_a_plausible_issue_rate():
    lib = kl.load()
    out = (ctypes.c_double * 2)()
    kl.check(lib.kh_probe_mfma_valu(1, 1, 0, 1, out), "kh_probe_mfma_valu")
    # a 32x32x2 fp32 MFMA keeps the matrix core 64 cycles at full rate
    assert 55.0 < out[0] < 200.0 and 0.5 < out[1] < 3.5
    kl.check(lib.kh_probe_mfma_valu(2, 8, 16, 2, out), "kh_probe_mfma_valu")
    assert 20.0 < out[0] < 400.0
    with pytest.raises(ValueError):
        kl.check(lib.kh_probe_mfma_valu(3, 3, 3, 1, out), "kh_probe_mfma_valu")
    with pytest.raises(ValueError):
        kl.check(lib.kh_probe_mfma_valu(1, 1, 0, 4, out), "kh_probe_mfma_valu")
