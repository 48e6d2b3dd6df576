"""q/k Gemma RMS norm + partial rotary embedding + KV store, restated in numpy.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the
HIP entry point ``nq_qk_norm_rope_store``, never a product path.

What it restates (the part of ``Qwen3_5Attention.forward`` between the
projections and the attention call, models/qwen3_5.py:135-139):

* ``GemmaRMSNorm.rms_forward`` (layers/layernorm.py:81-91)::

      x = x.float(); var = x.pow(2).mean(-1, keepdim=True)
      x = x * torch.rsqrt(var + eps)
      x = x.to(orig_dtype) * (1.0 + self.weight)

  The method is ``@torch.compile``d.  Inductor keeps the explicit cast
  ``x.to(orig_dtype)`` (a rounding to the tensor's dtype) but computes
  ``1.0 + weight`` and the product in float32, rounding once when the result
  is stored.  ``gemma_rms_norm`` follows that.  Eager PyTorch would also
  round ``1.0 + weight``; the two agree whenever ``1 + w`` is representable in
  the dtype, and otherwise differ by at most one unit in the last place.
  ``rsqrt`` is taken as ``1 / sqrt`` with IEEE float32 sqrt and division.
  The float32 sum of squares needs an order; ``sum_squares`` fixes the one
  the HIP kernel uses (8-element left-to-right partial sums, then a butterfly
  tree over the partials), one valid order for the reference's ``mean``,
  whose compiled reduction order is Inductor's and is not pinned at the
  last bit.  With that order and every operation rounded on its own, the
  kernel must match this oracle bit for bit.

* ``InterleavedMRoPE.__init__`` / ``forward`` (layers/rotary_embedding.py:
  83-123) and ``apply_rotary_emb`` (:6-14): only the first ``rotary_dim``
  dims rotate; with ``c, s = cos_sin_cache[pos]`` split in halves and
  ``x1, x2`` the halves of the rotary slice (float32)::

      y1 = x1 * c - x2 * s;  y2 = x2 * c + x1 * s;  cast back to the dtype

  The mrope sections are a numerical identity for text positions (all three
  position streams equal, :76-80), so the table is the plain 1-D one.

* ``store_kvcache(key, value, ...)`` (layers/attention.py:62-63) of the
  rotated key and the raw value, through ``oracle.paged.store_kvcache`` (or the
  fp8 quantizer of ``oracle.fp8`` for an e4m3fn cache).

Arrays are float32 holding values representable in ``dtype``
("bf16" | "f16" | "f32").
"""
from __future__ import annotations

import numpy as np

from . import fp8 as _fp8
from .paged import store_kvcache as _store

F32 = np.float32


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` (nearest even), returned as float32."""
    x = np.asarray(x, dtype=F32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(F32)
    if dtype != "bf16":
        raise ValueError(dtype)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(F32).copy()
    nan = np.isnan(x)
    out[nan] = x[nan]
    return out


def rope_cache(rotary_dim: int, max_position: int, base: float) -> np.ndarray:
    """``cos_sin_cache`` of layers/rotary_embedding.py:96-102 as [max_position, R].

    inv_freq = 1 / base ** (arange(0, R, 2) / R), freqs = t x inv_freq, all
    float32; the row is the R/2 cosines followed by the R/2 sines.
    """
    R = rotary_dim
    inv_freq = (F32(1.0) / (F32(base) ** (np.arange(0, R, 2, dtype=F32) / F32(R)))).astype(F32)
    t = np.arange(max_position, dtype=F32)
    freqs = np.outer(t, inv_freq).astype(F32)
    return np.concatenate([np.cos(freqs), np.sin(freqs)], axis=-1).astype(F32)


def sum_squares(x: np.ndarray, group: int = 8) -> np.ndarray:
    """float32 sum of x*x over the last axis in a fixed order: partial sums of
    ``group`` consecutive squares, left to right, then a butterfly over the
    L = D/group partials (p[i] += p[i ^ off] for off = L/2, ..., 1, after
    which every partial holds the total).  Keeps the reduced axis (size 1)."""
    xf = np.asarray(x, dtype=F32)
    d = xf.shape[-1]
    sq = (xf * xf).reshape(*xf.shape[:-1], d // group, group)
    p = sq[..., 0].copy()
    for i in range(1, group):
        p = p + sq[..., i]
    lanes = np.arange(d // group)
    off = (d // group) // 2
    while off >= 1:
        p = p + p[..., lanes ^ off]
        off //= 2
    return p[..., :1]


def gemma_rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, dtype: str,
                   weight_offset: float = 1.0) -> np.ndarray:
    """layers/layernorm.py:81-91 over the last axis (see the module docstring)."""
    xf = np.asarray(x, dtype=F32)
    var = sum_squares(xf) * F32(1.0 / xf.shape[-1])
    r = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    n = round_to(xf * r, dtype)
    w = np.asarray(weight, dtype=F32) + F32(weight_offset)
    return round_to(n * w, dtype)


def apply_partial_rope(x: np.ndarray, cos_sin: np.ndarray, rotary_dim: int, dtype: str) -> np.ndarray:
    """layers/rotary_embedding.py:6-14 and :111-119 for x [N, H, D].

    ``cos_sin`` [N, R] holds each token's table row (already gathered by
    position).  Dims >= R pass through.
    """
    R = rotary_dim
    if R == 0:
        return np.asarray(x, dtype=F32).copy()
    half = R // 2
    c = cos_sin[:, None, :half].astype(F32)
    s = cos_sin[:, None, half:R].astype(F32)
    x1 = x[..., :half].astype(F32)
    x2 = x[..., half:R].astype(F32)
    y1 = x1 * c - x2 * s
    y2 = x2 * c + x1 * s
    return np.concatenate([round_to(y1, dtype), round_to(y2, dtype), x[..., R:].astype(F32)], axis=-1)


def qk_norm_rope(q, k, positions, cos_sin_cache, rotary_dim, q_weight, k_weight, eps, dtype,
                 weight_offset: float = 1.0):
    """q [N, Hq, D], k [N, Hkv, D] -> (q_out, k_out), models/qwen3_5.py:135-137.

    Rows whose position lies outside the table are NaN (the reference's
    table index would fail there).
    """
    positions = np.asarray(positions, dtype=np.int64)
    max_pos = cos_sin_cache.shape[0] if rotary_dim else np.iinfo(np.int64).max
    bad = (positions < 0) | (positions >= max_pos)
    rows = np.zeros((len(positions), rotary_dim), dtype=F32)
    if rotary_dim:
        rows = cos_sin_cache[np.where(bad, 0, positions)][:, :rotary_dim]
    qn = gemma_rms_norm(q, q_weight, eps, dtype, weight_offset)
    kn = gemma_rms_norm(k, k_weight, eps, dtype, weight_offset)
    q_out = apply_partial_rope(qn, rows, rotary_dim, dtype)
    k_out = apply_partial_rope(kn, rows, rotary_dim, dtype)
    q_out[bad] = np.nan
    k_out[bad] = np.nan
    return q_out, k_out


def store_rows(k_out, v, k_cache, v_cache, slot_mapping, k_scale=None, v_scale=None):
    """The store after the norm and rotation (layers/attention.py:62-63).

    Same-dtype caches (float32 arrays) receive the rows; fp8 caches (uint8
    code arrays) receive ``fp8.quantize`` of them with the per-head scales.
    Slots outside [0, num_slots) are skipped.
    """
    if k_cache.dtype == np.uint8:
        n, hkv, d = k_out.shape
        slots = np.asarray(slot_mapping, dtype=np.int64)
        num_slots = k_cache.reshape(-1, hkv * d).shape[0]
        ok = (slots >= 0) & (slots < num_slots)
        kc = k_cache.reshape(-1, hkv, d)
        vc = v_cache.reshape(-1, hkv, d)
        kc[slots[ok]] = _fp8.quantize(k_out[ok], k_scale)
        vc[slots[ok]] = _fp8.quantize(v[ok], v_scale)
        return
    _store(k_out, v, k_cache, v_cache, slot_mapping)
