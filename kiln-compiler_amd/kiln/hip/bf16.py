"""bf16 copies of GEMM weights for the bf16-input GEMM variants.

The library's bf16 GEMM reads B as a bf16 copy of a constant in [batch][N][K']
layout (K' = K rounded up to 8, zero padded), so each lane's 8 K values are
one 16-byte chunk. The three-pass variant (allow_tf32) reads [batch][N][2K']:
each row holds bf16(w), then bf16(w - bf16(w)). The copy is made once, on the host, when the executable is
built - the analogue of the reference's freeze-time constant folding of W^T
(kiln/passes/freeze.py:45-75), with a precision change.
"""

from __future__ import annotations

import numpy as np


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest, ties to even.

    Adds 0x7FFF plus the lowest kept bit to the float32 pattern and keeps the
    upper 16 bits; values that round past the largest finite bf16 become inf.
    NaNs stay NaN (the quiet bit is set so a payload in the dropped bits
    cannot turn one into inf).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    out = ((u + (((u >> 16) & np.uint32(1)) + np.uint32(0x7FFF))) >> 16).astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | np.uint32(0x0040)).astype(np.uint16)
    return out


def padded_k(k: int) -> int:
    return (k + 7) // 8 * 8


def weight_copy(data: np.ndarray, offset: int, strides, batch: int, k: int, n: int) -> np.ndarray:
    """The bf16 [batch][N][K'] copy of the [batch, K, N] view (element offset,
    strides over (b, k, n)) of a constant, as uint16 bit patterns."""
    flat = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    sb, sk, sn = (int(s) for s in strides)
    idx = (offset + np.arange(batch)[:, None, None] * sb + np.arange(n)[None, :, None] * sn
           + np.arange(k)[None, None, :] * sk)
    out = np.zeros((batch, n, padded_k(k)), np.uint16)
    out[:, :, :k] = bf16_bits(flat[idx])
    return out


def bf16_value(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> the float32 values they encode."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def weight_copy_x3(data: np.ndarray, offset: int, strides, batch: int, k: int, n: int) -> np.ndarray:
    """The three-pass [batch][N][2K'] copy of the same view: hi = bf16(w) in
    [0, K'), lo = bf16(w - hi) in [K', 2K') (w - hi is exact in float32; a
    non-finite hi keeps lo 0), as uint16 bit patterns."""
    hi = weight_copy(data, offset, strides, batch, k, n)
    flat = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    sb, sk, sn = (int(s) for s in strides)
    idx = (offset + np.arange(batch)[:, None, None] * sb + np.arange(n)[None, :, None] * sn
           + np.arange(k)[None, None, :] * sk)
    w = flat[idx]
    hv = bf16_value(hi[:, :, :k])
    with np.errstate(invalid="ignore", over="ignore"):
        rest = np.where(np.isfinite(hv), w - hv, np.float32(0.0)).astype(np.float32)
    kp = padded_k(k)
    out = np.zeros((batch, n, 2 * kp), np.uint16)
    out[:, :, :kp] = hi
    out[:, :, kp:kp + k] = bf16_bits(rest)
    return out
