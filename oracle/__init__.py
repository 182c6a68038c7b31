"""CPU oracle for Kiln's GPU hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product (kiln/) never
imports it.

  * ``kiln_oracle.c`` (via ``lib()``): bf16 rounding and float64 restatements of GELU, bias+GELU,
    LayerNorm, softmax, strided batched matmul, Linear + epilogue and the
    GPT-2 block, following the reference's op definitions and decompositions
    (file:line citations in the C source).
  * ``interp.py``: a float64 NumPy interpreter of Kiln IR graphs (the
    reference's op table, kiln/ir/ops.py:48-188), for arbitrary fused graphs.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkiln_oracle.so"

_lib = None


def lib():
    """The compiled C oracle (built on first use if missing)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build

            build()
        L = ctypes.CDLL(str(LIB_PATH))
        f, i64, dbl, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int
        L.ko_gelu.argtypes = [f, i64, i, f]
        L.ko_bias_gelu.argtypes = [f, f, i64, i64, i, f]
        L.ko_layernorm.argtypes = [f, f, f, dbl, i64, i64, f]
        L.ko_softmax.argtypes = [f, dbl, i64, i64, f]
        L.ko_matmul.argtypes = [f, i64, i64, i64, f, i64, i64, i64, i64, i64, i64, i64, f]
        L.ko_linear.argtypes = [f, f, f, f, i, i64, i64, i64, f]
        L.ko_block.argtypes = [f, i64, i64, i64] + [f] * 12 + [f]
        L.ko_bf16_round.argtypes = [f, i64, f]
        for name in ("ko_bf16_round", "ko_gelu", "ko_bias_gelu", "ko_layernorm", "ko_softmax", "ko_matmul", "ko_linear", "ko_block"):
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data


def bf16_round(x):
    """Nearest bfloat16 value of each element (ties to even), as float32."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().ko_bf16_round(_p(x), x.size, _p(out))
    return out


def gelu(x, approximate="none"):
    x = _f32(x)
    out = np.empty_like(x)
    lib().ko_gelu(_p(x), x.size, int(approximate == "tanh"), _p(out))
    return out


def bias_gelu(x, b, approximate="tanh"):
    x, b = _f32(x), _f32(b)
    out = np.empty_like(x)
    lib().ko_bias_gelu(_p(x), _p(b), x.shape[0], x.shape[1], int(approximate == "tanh"), _p(out))
    return out


def layernorm(x, gamma=None, beta=None, eps=1e-5):
    x = _f32(x)
    g = None if gamma is None else _f32(gamma)
    b = None if beta is None else _f32(beta)
    inner = x.shape[-1]
    out = np.empty_like(x)
    lib().ko_layernorm(_p(x), _p(g), _p(b), eps, x.size // max(inner, 1), inner, _p(out))
    return out


def softmax(x, scale=1.0):
    x = _f32(x)
    inner = x.shape[-1]
    out = np.empty_like(x)
    lib().ko_softmax(_p(x), scale, x.size // max(inner, 1), inner, _p(out))
    return out


def matmul(a, b):
    """a [..., M, K] @ b [..., K, N] for rank 2 or 3 (batch dims equal)."""
    a, b = _f32(a), _f32(b)
    a3 = a.reshape(-1, *a.shape[-2:])
    b3 = b.reshape(-1, *b.shape[-2:])
    batch, M, K = a3.shape
    N = b3.shape[-1]
    out = np.empty((batch, M, N), np.float32)
    lib().ko_matmul(_p(a3), M * K, K, 1, _p(b3), K * N, N, 1, batch, M, N, K, _p(out))
    return out.reshape(*a.shape[:-1], N)


def linear(x, wt, bias=None, residual=None, act="none"):
    """act(x @ wt + bias) + residual with wt = W^T [K, N]."""
    x, wt = _f32(x), _f32(wt)
    M, K = x.shape
    N = wt.shape[1]
    bias = None if bias is None else _f32(bias)
    residual = None if residual is None else _f32(residual)
    out = np.empty((M, N), np.float32)
    code = {"none": 0, "tanh": 1, "erf": 2}[act]
    lib().ko_linear(_p(x), _p(wt), _p(bias), _p(residual), code, M, N, K, _p(out))
    return out


def block(x, params, nh):
    """GPT-2 block forward; params: dict of numpy arrays named as the torch
    module's state dict (weights [out, in] as in nn.Linear)."""
    x = _f32(x)
    T, d = x.shape
    P = {k: _f32(v) for k, v in params.items()}
    wt = lambda name: _f32(P[name].T)
    keep = [wt("c_attn.weight"), wt("c_proj.weight"), wt("fc.weight"), wt("proj.weight")]
    out = np.empty_like(x)
    lib().ko_block(_p(x), T, d, nh, _p(P["ln1.weight"]), _p(P["ln1.bias"]), _p(keep[0]), _p(P["c_attn.bias"]),
                   _p(keep[1]), _p(P["c_proj.bias"]), _p(P["ln2.weight"]), _p(P["ln2.bias"]), _p(keep[2]),
                   _p(P["fc.bias"]), _p(keep[3]), _p(P["proj.bias"]), _p(out))
    return out
