"""Paged KV store and paged attention in float64 numpy (oracle; test only).

Restates the arithmetic of the reference's paged attention path:

* ``store_kvcache``  -- layers/attention.py:10-40 (Triton scatter).
* ``paged_decode``   -- layers/attention.py:71-74, i.e. flash_attn's
  ``flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
  cache_seqlens=context_lens, block_table=block_tables, causal=True)``.
* ``varlen_prefill`` -- layers/attention.py:64-70, i.e. flash_attn's
  ``flash_attn_varlen_func(..., causal=True, block_table=...)`` with the
  K/V source switch of :65-66 (whole paged cache when ``block_tables`` is set).

Conventions fixed by the reference's call sites:

* cache layout ``[num_blocks, block_size, Hkv, D]`` (engine/model_runner.py:198);
  key ``j`` of sequence ``s`` lives at row
  ``block_tables[s, j // block_size] * block_size + j % block_size``.
* GQA: query head ``h`` reads kv head ``h // (Hq // Hkv)`` (flash_attn's
  grouping; the caller builds contiguous head groups, models/qwen3_5.py:65-68).
* causal masking is aligned to the bottom-right corner: with
  ``P = Lk - Lq``, query row ``i`` sees keys ``j <= i + P`` (flash_attn >= 2.1
  semantics; prefix-cached prefill relies on it, engine/model_runner.py:252-259).
* decode: ``context_lens[b]`` already counts the token just stored
  (engine/decode_init.py:30-36); rows with ``context_len <= 0`` (graph padding,
  engine/model_runner.py:332) produce zeros here, a build convention -- the
  reference discards those rows.
"""
from __future__ import annotations

import numpy as np


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """Scatter new K/V rows into the paged caches in place (byte-exact).

    layers/attention.py:21-30: for token ``i`` with ``slot = slot_mapping[i]``,
    ``k_cache.flat[slot*Hkv*D : (slot+1)*Hkv*D] = key[i]`` (same for V); a
    slot of -1 skips the token (:23).  Any negative slot or a slot past the
    pool is skipped as well (the build bounds-checks; the reference would
    write out of bounds).  Works for any element type because it is a copy.
    """
    n = key.shape[0]
    kc = k_cache.reshape(-1, key.shape[1] * key.shape[2])
    vc = v_cache.reshape(-1, value.shape[1] * value.shape[2])
    slots = np.asarray(slot_mapping).astype(np.int64).reshape(-1)
    assert slots.shape[0] == n
    ok = (slots >= 0) & (slots < kc.shape[0])
    kc[slots[ok]] = key.reshape(n, -1)[ok]
    vc[slots[ok]] = value.reshape(n, -1)[ok]
    return k_cache, v_cache


def gather_keys(cache, table_row, n_keys):
    """Rows 0..n_keys-1 of one sequence through its block-table row."""
    bs = cache.shape[1]
    nblk = -(-int(n_keys) // bs)
    blocks = np.asarray(table_row[:nblk]).astype(np.int64)
    assert np.all(blocks >= 0), "block table entry needed but -1"
    return cache[blocks].reshape(-1, cache.shape[2], cache.shape[3])[:n_keys]


def _softmax_attend(qh, kh, vh, scale, mask=None):
    """qh [M, D], kh [N, D], vh [N, D] (float64) -> [M, D]; masked rows -> 0."""
    s = (qh @ kh.T) * scale
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(mx)
    mx = np.where(empty, 0.0, mx)
    p = np.exp(s - mx)
    den = p.sum(axis=-1, keepdims=True)
    den = np.where(den == 0.0, 1.0, den)
    o = (p / den) @ vh
    return np.where(empty, 0.0, o)


def paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale,
                 k_scale=None, v_scale=None):
    """q [B, Hq, D]; caches [NB, BS, Hkv, D] (float values) -> [B, Hq, D] f64.

    ``k_scale`` / ``v_scale`` ([Hkv]) multiply the cached values of each kv
    head (the fp8 dequantization), i.e. attention runs over
    ``k_cache * k_scale`` and ``v_cache * v_scale``.
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, D = q.shape
    hkv = k_cache.shape[2]
    g = Hq // hkv
    assert g * hkv == Hq
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        K = gather_keys(k_cache, block_tables[b], ctx).astype(np.float64)
        V = gather_keys(v_cache, block_tables[b], ctx).astype(np.float64)
        for h in range(hkv):
            kh, vh = K[:, h], V[:, h]
            if k_scale is not None:
                kh = kh * float(k_scale[h])
            if v_scale is not None:
                vh = vh * float(v_scale[h])
            out[b, h * g:(h + 1) * g] = _softmax_attend(q[b, h * g:(h + 1) * g], kh, vh, scale)
    return out


def varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_tables=None,
                   rows=None, k_scale=None, v_scale=None):
    """Causal varlen attention, bottom-right aligned, float64.

    q [Tq, Hq, D] packed by ``cu_seqlens_q``.  Without ``block_tables`` the
    keys are packed ``k, v [Tk, Hkv, D]`` by ``cu_seqlens_k``; with it ``k, v``
    are the paged caches ``[NB, BS, Hkv, D]`` and sequence ``s`` reads its
    first ``Lk`` keys through ``block_tables[s]`` (layers/attention.py:65-66).
    ``rows`` optionally restricts the computation to a subset of global query
    rows (the others stay zero) so large cases can be spot-checked.
    """
    q = np.asarray(q, dtype=np.float64)
    Tq, Hq, D = q.shape
    hkv = k.shape[-2]
    g = Hq // hkv
    cq = np.asarray(cu_seqlens_q).astype(np.int64)
    ck = np.asarray(cu_seqlens_k).astype(np.int64)
    out = np.zeros((Tq, Hq, D), dtype=np.float64)
    want = None if rows is None else np.zeros(Tq, dtype=bool)
    if want is not None:
        want[np.asarray(rows, dtype=np.int64)] = True
    for s in range(len(cq) - 1):
        q0, q1 = cq[s], cq[s + 1]
        lq, lk = q1 - q0, ck[s + 1] - ck[s]
        if lq <= 0:
            continue
        local = np.arange(lq)
        if want is not None:
            local = local[want[q0:q1]]
            if local.size == 0:
                continue
        if block_tables is None:
            K = np.asarray(k[ck[s]:ck[s + 1]], dtype=np.float64)
            V = np.asarray(v[ck[s]:ck[s + 1]], dtype=np.float64)
        else:
            K = gather_keys(k, block_tables[s], lk).astype(np.float64)
            V = gather_keys(v, block_tables[s], lk).astype(np.float64)
        p = lk - lq
        mask = np.arange(lk)[None, :] <= (local[:, None] + p)
        for h in range(hkv):
            kh, vh = K[:, h], V[:, h]
            if k_scale is not None:
                kh = kh * float(k_scale[h])
            if v_scale is not None:
                vh = vh * float(v_scale[h])
            for hq in range(h * g, (h + 1) * g):
                out[q0 + local, hq] = _softmax_attend(q[q0 + local, hq], kh, vh, scale, mask)
    return out
