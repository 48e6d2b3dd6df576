"""OCP float8 e4m3fn codec in numpy (oracle; test infrastructure only).

The reference has no fp8 KV cache (its roadmap item, README.md:30, is
unchecked); the fp8 variant of the path is specified by the build's target:
K/V are quantized per (layer, kv_head) with ``scale = absmax / 448`` and the
cache stores e4m3fn codes.  The quantizer restated here is the exact
arithmetic the HIP store kernel performs, so the two must agree bit for bit:

    inv   = float32(1) / float32(scale)          (IEEE division, RN)
    y     = float32(x) * inv                     (IEEE multiply, RN)
    y     = min(max(y, -448), 448)               (saturate)
    code  = round-to-nearest-even of y onto the e4m3fn grid

e4m3fn: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits, no
infinities, code 0x7F / 0xFF is NaN, largest finite value 448 = 1.75 * 2^8,
smallest subnormal 2^-9.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def _positive_grid() -> np.ndarray:
    """Values of codes 0..126 (all non-negative finite e4m3fn), ascending."""
    vals = []
    for c in range(127):
        e, m = c >> 3, c & 7
        if e == 0:
            vals.append(m / 8.0 * 2.0 ** -6)
        else:
            vals.append((1.0 + m / 8.0) * 2.0 ** (e - 7))
    return np.asarray(vals, dtype=np.float64)


_GRID = _positive_grid()


def decode_e4m3fn(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (NaN for 0x7F/0xFF)."""
    c = np.asarray(codes, dtype=np.uint8)
    mag = c & 0x7F
    out = np.where(mag == 0x7F, np.nan, _GRID[np.minimum(mag, 126)])
    out = np.where(c & 0x80, -out, out)
    return out.astype(np.float32)


def encode_e4m3fn(y: np.ndarray) -> np.ndarray:
    """float32 values already inside [-448, 448] (or NaN) -> uint8 codes, RNE.

    Ties go to the code with an even mantissa, i.e. the even code, because
    codes are monotone in magnitude.  NaN maps to 0x7F with its sign bit.
    """
    y = np.asarray(y, dtype=np.float32)
    sign = (y.view(np.uint32) >> 31).astype(np.uint8)
    a = np.abs(y.astype(np.float64))
    nan = np.isnan(a)
    a = np.where(nan, 0.0, a)
    if np.any(a > E4M3_MAX):
        raise ValueError("encode_e4m3fn expects saturated input (|y| <= 448)")
    hi = np.searchsorted(_GRID, a, side="left")        # first grid value >= a
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    v_hi, v_lo = _GRID[hi], _GRID[lo]
    d_hi, d_lo = v_hi - a, a - v_lo
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(a == v_hi, hi, np.where(pick_hi, hi, lo)).astype(np.uint8)
    code = np.where(nan, np.uint8(0x7F), code)
    return (code | (sign << 7)).astype(np.uint8)


def inv_scale(scale: np.ndarray) -> np.ndarray:
    """float32 reciprocal the store kernel multiplies by (IEEE division)."""
    s = np.asarray(scale, dtype=np.float32)
    return (np.float32(1.0) / s).astype(np.float32)


def quantize(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """x [..., Hkv, D] float32, scale [Hkv] float32 -> uint8 e4m3fn codes."""
    x = np.asarray(x, dtype=np.float32)
    inv = inv_scale(scale)[:, None]
    y = (x * inv).astype(np.float32)
    y = np.minimum(np.maximum(y, np.float32(-E4M3_MAX)), np.float32(E4M3_MAX))
    return encode_e4m3fn(y)


def absmax_scale(x: np.ndarray) -> np.ndarray:
    """Per-kv-head scale = absmax / 448 over every axis but the head axis.

    ``x`` is [..., Hkv, D]; the result is float32 [Hkv].  A head that is all
    zeros gets scale 1 so the reciprocal stays finite.
    """
    x = np.asarray(x, dtype=np.float32)
    hk = x.shape[-2]
    amax = np.abs(x.reshape(-1, hk, x.shape[-1])).max(axis=(0, 2))
    s = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    return np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
