"""Python entry points of the HIP paged attention kernels.

Thin wrappers over the C ABI (include/nq_attn.h): they check shapes and
strides, pick dtype codes, pass raw device pointers and torch's current
stream, and raise ``RuntimeError`` on a non-zero status.  The argument names
and meanings follow the calls the reference makes:

* ``store_kvcache``   -- layers/attention.py:33-40
* ``varlen_prefill``  -- flash_attn_varlen_func at layers/attention.py:67-70
* ``paged_decode``    -- flash_attn_with_kvcache at layers/attention.py:72-74
* ``prepare_decode``  -- engine/decode_init.py:39-65
* ``qk_norm_rope_store`` -- models/qwen3_5.py:135-137 + layers/attention.py:63
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib
from ._lib import check, dtype_code, lib, ptr, require_cuda, stream_of

# Persistent device buffers of the kernels, one per (device, stream): calls
# on one stream are ordered, so they may share a buffer; calls on different
# streams get their own.  A buffer that has to grow is replaced, but the old
# one is kept alive (``_retired``): a HIP graph captured earlier may still
# hold its address, and replays must keep writing into valid memory.  The
# tables therefore grow with the number of streams ever used: callers should
# launch from a fixed set of streams, and ``release_workspaces`` frees every
# buffer once no captured graph that used them will be replayed.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_prefill_queues: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []
_DEBUG_QUEUE = os.environ.get("NQ_DEBUG_PREFILL_QUEUE", "0") not in ("", "0")


def _key(device) -> tuple[int, int]:
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return idx, torch.cuda.current_stream(idx).cuda_stream


def _grow(table, key, nbytes, dtype, device, zero=False):
    """The buffer of ``key`` in ``table`` with at least ``nbytes`` bytes;
    grows geometrically, retiring (never freeing) the buffer it replaces."""
    cur = table.get(key)
    if cur is not None and cur.numel() * cur.element_size() >= nbytes:
        return cur
    have = 0 if cur is None else cur.numel() * cur.element_size()
    size = max(nbytes, 2 * have, 1 << 20)
    item = torch.empty((), dtype=dtype).element_size()
    n = (size + item - 1) // item
    buf = torch.zeros(n, dtype=dtype, device=device) if zero else torch.empty(n, dtype=dtype, device=device)
    if cur is not None:
        _retired.append(cur)
    table[key] = buf
    return buf


def release_workspaces(device=None) -> int:
    """Drop the kernels' per-stream buffers (decode split-K workspaces,
    prefill queue counters) and every retired buffer, of ``device`` or of
    all devices; returns how many were dropped.  Only safe once no HIP graph
    captured with them will be replayed again: a replay would write freed
    memory.  Later calls allocate fresh buffers (the prefill counters start
    at zero again)."""
    idx = None if device is None else _key(device)[0]
    n = 0
    for table in (_workspaces, _prefill_queues):
        for key in [k for k in table if idx is None or k[0] == idx]:
            del table[key]
            n += 1
    keep = [t for t in _retired if idx is not None and t.device.index != idx]
    n += len(_retired) - len(keep)
    _retired[:] = keep
    return n


def store_kvcache(key, value, k_cache, v_cache, slot_mapping, k_scale=None, v_scale=None):
    """Scatter ``key/value [N, Hkv, D]`` into cache rows ``slot_mapping [N]``.

    Same-dtype caches get a byte-exact copy; a ``float8_e4m3fn`` cache is
    quantized with ``k_scale/v_scale [Hkv]`` (``x * (1/scale)``, saturate to
    +-448, round to nearest even).
    """
    require_cuda(key, value, k_cache, v_cache, slot_mapping, what="store_kvcache")
    n, hkv, d = key.shape
    if slot_mapping.dtype != torch.int32:
        raise RuntimeError("store_kvcache: slot_mapping must be int32")
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    if fp8 and (k_scale is None or v_scale is None):
        raise RuntimeError("store_kvcache: an fp8 cache needs k_scale and v_scale")
    if not fp8 and k_cache.dtype != key.dtype:
        raise RuntimeError(f"store_kvcache: cache dtype {k_cache.dtype} != key dtype {key.dtype}")
    num_slots = k_cache.numel() // (hkv * d)
    rc = lib().nq_store_kvcache(
        ptr(key), key.stride(0), ptr(value), value.stride(0), ptr(k_cache), ptr(v_cache),
        ptr(slot_mapping), n, num_slots, hkv, d, dtype_code(key.dtype), dtype_code(k_cache.dtype),
        ptr(k_scale) if fp8 else None, ptr(v_scale) if fp8 else None, stream_of(key))
    check(rc, "store_kvcache")


def decode_plan(batch, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size, kv_dtype):
    """(num_splits, split_tokens) chosen from host-known shapes only."""
    ns, st = ctypes.c_int(), ctypes.c_int()
    rc = lib().nq_decode_plan(batch, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size,
                              dtype_code(kv_dtype), ctypes.byref(ns), ctypes.byref(st))
    check(rc, "decode_plan")
    return ns.value, st.value


def decode_schedule(batch, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size, kv_dtype,
                    num_splits, workspace_bytes) -> str:
    """``"stream-K"`` or ``"split-K"``: the schedule ``nq_paged_decode``
    takes for these shapes, plan and workspace size (a single split reports
    ``"split-K"``)."""
    rc = lib().nq_decode_schedule(batch, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                                  dtype_code(kv_dtype), num_splits, int(workspace_bytes))
    if rc < 0:
        check(rc, "decode_schedule")
    return "stream-K" if rc == 1 else "split-K"


def decode_workspace(device, nbytes: int) -> torch.Tensor | None:
    """Persistent split-K workspace of at least ``nbytes`` for the current
    stream of ``device``.

    Kept across calls so a captured HIP graph keeps a fixed pointer.  Growing
    it never frees the old buffer (a graph may hold it); growing it inside a
    capture allocates from the capture's pool, which torch keeps alive with
    the graph.  ``reserve_decode_workspace`` sizes it once up front.
    """
    if nbytes <= 0:
        return None
    return _grow(_workspaces, _key(device), nbytes, torch.uint8, device)


def reserve_decode_workspace(device, max_batch, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size,
                             head_dim, kv_dtype) -> int:
    """Size the current stream's split-K workspace for the largest decode
    the caller will run (batch ``max_batch``, tables ``max_blocks_per_seq``
    wide); returns its bytes.  Every batch up to ``max_batch`` then fits
    without growing.  The plan's split count falls as the batch grows, so
    every batch size is checked."""
    need = 0
    for b in range(1, int(max_batch) + 1):
        ns, _ = decode_plan(b, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size, kv_dtype)
        need = max(need, lib().nq_decode_workspace_bytes(b, num_q_heads, head_dim, ns))
    if need > 0:
        decode_workspace(device, need)
    return need


def prefill_workspace(device) -> torch.Tensor:
    """Work-queue counters of the prefill kernel for the current stream of
    ``device``.

    Zeroed once here; every completed prefill call leaves them zero again, so
    the same tensor serves every later call on that stream (and graph
    replays).  Each stream has its own, so launches on different streams
    never share counters.  With ``NQ_DEBUG_PREFILL_QUEUE=1`` every prefill
    synchronizes and checks that it left them zero.
    """
    return _grow(_prefill_queues, _key(device), lib().nq_prefill_workspace_bytes(), torch.int32, device,
                 zero=True)


def _check_queue_zero(ws):
    torch.cuda.current_stream(ws.device).synchronize()
    if int(ws.count_nonzero()) != 0:
        raise RuntimeError("varlen_prefill: the work-queue counters are not zero after the launch "
                           f"({ws[:16].tolist()}); a launch on this stream did not complete")


def _gate3(gate, n, hq, d, what):
    g3 = gate.squeeze(1) if gate.dim() == 4 else gate
    if g3.shape != (n, hq, d) or g3.stride(-1) != 1:
        raise RuntimeError(f"{what}: gate must be [N, Hq, D] with a contiguous last dim")
    return g3


def paged_decode(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale,
                 k_scale=None, v_scale=None, out=None, gate=None, k=None, v=None, slot_mapping=None):
    """Paged decode attention: ``q [B, 1, Hq, D]`` (or ``[B, Hq, D]``).

    Returns ``out`` shaped like ``q`` (``[B, 1, Hq, D]`` as
    flash_attn_with_kvcache does).  ``cache_seqlens [B] int32`` counts the
    cached tokens including the new one; ``block_table [B, W] int32``.
    With ``gate [B, Hq, D]`` (Qwen3.5's output gate, models/qwen3_5.py:142)
    the output is ``out * sigmoid(gate)``, applied in the kernel's store.
    With ``k, v [B, Hkv, D]`` and ``slot_mapping [B] int32`` the new token is
    stored in the same launch (``nq_paged_decode_store``): the result and the
    cache equal ``store_kvcache`` followed by this call when each
    ``slot_mapping[b]`` is -1 or the slot of token ``cache_seqlens[b] - 1``
    of ``block_table[b]`` (what prepare_decode writes).
    """
    require_cuda(q, k_cache, v_cache, cache_seqlens, block_table, what="paged_decode")
    q3 = q.squeeze(1) if q.dim() == 4 else q
    if q3.dim() != 3 or q3.stride(-1) != 1:
        raise RuntimeError("paged_decode: q must be [B, 1, Hq, D] / [B, Hq, D] with a contiguous last dim")
    B, hq, d = q3.shape
    nb, bs, hkv, d2 = k_cache.shape
    if d2 != d or v_cache.shape != k_cache.shape:
        raise RuntimeError("paged_decode: cache shape mismatch")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError("paged_decode: caches must be contiguous [num_blocks, block_size, Hkv, D]")
    if cache_seqlens.dtype != torch.int32 or block_table.dtype != torch.int32:
        raise RuntimeError("paged_decode: cache_seqlens and block_table must be int32")
    if block_table.stride(-1) != 1:
        raise RuntimeError("paged_decode: block_table rows must be contiguous")
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    o3 = out.squeeze(1) if out.dim() == 4 else out
    W = block_table.shape[1]
    ns, st = decode_plan(B, hq, hkv, W, bs, k_cache.dtype)
    wsb = lib().nq_decode_workspace_bytes(B, hq, d, ns)
    ws = decode_workspace(q.device, wsb)
    args = (ptr(q3), q3.stride(0), q3.stride(1), ptr(k_cache), ptr(v_cache), ptr(block_table),
            block_table.stride(0), W, ptr(cache_seqlens), ptr(o3), o3.stride(0), o3.stride(1),
            B, hq, hkv, d, bs, nb, float(softmax_scale), ns, st, ptr(ws), 0 if ws is None else ws.numel(),
            dtype_code(q.dtype), dtype_code(k_cache.dtype), ptr(k_scale) if fp8 else None,
            ptr(v_scale) if fp8 else None)
    g3 = None
    if gate is not None:
        require_cuda(gate, what="paged_decode")
        if gate.dtype != q.dtype:
            raise RuntimeError("paged_decode: gate dtype must match q")
        g3 = _gate3(gate, B, hq, d, "paged_decode")
    if k is not None:
        require_cuda(k, v, slot_mapping, what="paged_decode")
        k3 = k.reshape(B, hkv, d) if k.dim() == 4 else k
        v3 = v.reshape(B, hkv, d) if v.dim() == 4 else v
        for t, what in ((k3, "k"), (v3, "v")):
            if t.shape != (B, hkv, d) or t.stride(-1) != 1 or t.stride(1) != d:
                raise RuntimeError(f"paged_decode: {what} must be [B, Hkv, D] with contiguous heads")
        if k3.dtype != v3.dtype or (not fp8 and k3.dtype != k_cache.dtype):
            raise RuntimeError("paged_decode: k/v dtype must match the cache (or be stored into an fp8 cache)")
        if slot_mapping.dtype != torch.int32 or slot_mapping.numel() != B:
            raise RuntimeError("paged_decode: slot_mapping must be int32 [B]")
        rc = lib().nq_paged_decode_store(
            ptr(q3), q3.stride(0), q3.stride(1), ptr(k_cache), ptr(v_cache), ptr(block_table),
            block_table.stride(0), W, ptr(cache_seqlens), ptr(k3), k3.stride(0), ptr(v3), v3.stride(0),
            ptr(slot_mapping), dtype_code(k3.dtype), ptr(o3), o3.stride(0), o3.stride(1),
            B, hq, hkv, d, bs, nb, float(softmax_scale), ns, st, ptr(ws), 0 if ws is None else ws.numel(),
            dtype_code(q.dtype), dtype_code(k_cache.dtype), ptr(k_scale) if fp8 else None,
            ptr(v_scale) if fp8 else None, ptr(g3) if g3 is not None else None,
            0 if g3 is None else g3.stride(0), 0 if g3 is None else g3.stride(1), stream_of(q))
    elif g3 is None:
        rc = lib().nq_paged_decode(*args, stream_of(q))
    else:
        rc = lib().nq_paged_decode_gated(*args, ptr(g3), g3.stride(0), g3.stride(1), stream_of(q))
    check(rc, "paged_decode")
    return out


def output_gate(out, gate):
    """In place: ``out [N, H, D] *= sigmoid(gate [N, H, D])`` with eager
    torch's 16-bit rounding (models/qwen3_5.py:140-142), one launch."""
    require_cuda(out, gate, what="output_gate")
    n, h, d = out.shape
    g3 = _gate3(gate, n, h, d, "output_gate")
    if out.stride(-1) != 1 or gate.dtype != out.dtype:
        raise RuntimeError("output_gate: out needs a contiguous last dim and the gate's dtype")
    check(lib().nq_output_gate(ptr(out), out.stride(0), out.stride(1), ptr(g3), g3.stride(0), g3.stride(1),
                               n, h, d, dtype_code(out.dtype), stream_of(out)), "output_gate")
    return out


def varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
                   causal=True, block_table=None, k_scale=None, v_scale=None, out=None, gate=None):
    """Causal varlen attention; ``q [Tq, Hq, D]`` -> ``[Tq, Hq, D]``.

    Without ``block_table``: ``k, v [Tk, Hkv, D]`` packed by ``cu_seqlens_k``.
    With it: ``k, v`` are the paged caches ``[num_blocks, block_size, Hkv, D]``.
    With ``gate [Tq, Hq, D]`` the output is ``out * sigmoid(gate)``
    (models/qwen3_5.py:142), applied in the kernel's output store (16-bit
    K/V) or by one in-place pass after it (fp8 K/V).
    """
    require_cuda(q, k, v, cu_seqlens_q, cu_seqlens_k, block_table, what="varlen_prefill")
    tq, hq, d = q.shape
    if q.stride(-1) != 1:
        raise RuntimeError("varlen_prefill: q needs a contiguous last dim")
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32:
        raise RuntimeError("varlen_prefill: cu_seqlens must be int32")
    n = cu_seqlens_q.numel() - 1
    if block_table is None:
        tk, hkv, d2 = k.shape
        if k.stride(-1) != 1 or k.stride(1) != d or k.stride(0) != v.stride(0) or v.stride(1) != d:
            raise RuntimeError("varlen_prefill: packed k/v must be [Tk, Hkv, D] with equal strides")
        kv_rs, bs, nb, W, bt_stride = k.stride(0), 0, 0, 0, 0
    else:
        if block_table.dtype != torch.int32 or block_table.stride(-1) != 1:
            raise RuntimeError("varlen_prefill: block_table must be int32 with contiguous rows")
        nb, bs, hkv, d2 = k.shape
        if not (k.is_contiguous() and v.is_contiguous()):
            raise RuntimeError("varlen_prefill: paged caches must be contiguous")
        kv_rs, W, bt_stride = hkv * d, block_table.shape[1], block_table.stride(0)
    if d2 != d:
        raise RuntimeError("varlen_prefill: head_dim mismatch")
    fp8 = k.dtype == torch.float8_e4m3fn
    if out is None:
        out = torch.empty(tq, hq, d, dtype=q.dtype, device=q.device)
    ws = prefill_workspace(q.device)
    args = (ptr(q), q.stride(0), q.stride(1), ptr(k), ptr(v), kv_rs, ptr(cu_seqlens_q), ptr(cu_seqlens_k),
            int(max_seqlen_q), int(max_seqlen_k), ptr(block_table), bt_stride, W, nb, ptr(out),
            out.stride(0), out.stride(1), n, hq, hkv, d, bs, float(softmax_scale), 1 if causal else 0,
            dtype_code(q.dtype), dtype_code(k.dtype), ptr(k_scale) if fp8 else None,
            ptr(v_scale) if fp8 else None, ptr(ws), ws.numel() * 4)
    if gate is None:
        rc = lib().nq_varlen_prefill(*args, stream_of(q))
    else:
        require_cuda(gate, what="varlen_prefill")
        if gate.dtype != q.dtype:
            raise RuntimeError("varlen_prefill: gate dtype must match q")
        g3 = _gate3(gate, tq, hq, d, "varlen_prefill")
        rc = lib().nq_varlen_prefill_gated(*args, ptr(g3), g3.stride(0), g3.stride(1), tq, stream_of(q))
    check(rc, "varlen_prefill")
    if _DEBUG_QUEUE:
        _check_queue_zero(ws)
    return out


def prepare_decode(sampled_token_ids, batch_slots, seq_lens, last_block_ids, input_ids, positions,
                   context_lens, slot_mapping, num_seqs, block_size):
    """Decode metadata kernel; same arguments as engine/decode_init.py:39-52."""
    require_cuda(seq_lens, last_block_ids, positions, context_lens, slot_mapping,
                 what="prepare_decode")
    rc = lib().nq_prepare_decode(
        ptr(sampled_token_ids), ptr(batch_slots), ptr(seq_lens), ptr(last_block_ids), ptr(input_ids),
        ptr(positions), ptr(context_lens), ptr(slot_mapping), int(num_seqs), int(block_size),
        stream_of(seq_lens))
    check(rc, "prepare_decode")


def qk_norm_rope_store(positions, query, key, value, q_weight, k_weight, eps, cos_sin_cache, rotary_dim,
                       k_cache=None, v_cache=None, slot_mapping=None, k_scale=None, v_scale=None,
                       weight_offset=1.0, q_out=None, k_out=None, _return_args=False):
    """Gemma RMS norm of ``query [N, Hq, D]`` / ``key [N, Hkv, D]``, rotary
    embedding of their first ``rotary_dim`` dims, and the KV store.

    One launch replacing ``q_norm``, ``k_norm`` and ``rotary_emb`` of
    models/qwen3_5.py:135-137 plus ``store_kvcache`` of layers/attention.py:63.
    ``query`` may be a strided view (the query half of ``q_proj``'s output).
    ``cos_sin_cache`` is the float32 table ``[max_position, (1,) rotary_dim]``
    (cosines, then sines); ``positions`` int64 ``[N]``.  Returns
    ``(q_out, k_out)``, new contiguous tensors unless given (passing the
    inputs rotates in place).  Without caches nothing is stored.
    ``_return_args`` returns the checked C-ABI argument tuple instead of
    launching (for timing loops that call the library directly).
    """
    require_cuda(positions, query, key, value, q_weight, k_weight, cos_sin_cache, k_cache, v_cache,
                 slot_mapping, what="qk_norm_rope_store")
    n, hq, d = query.shape
    n2, hkv, d2 = key.shape
    if n2 != n or d2 != d or query.stride(-1) != 1 or key.stride(-1) != 1 or key.stride(1) != d:
        raise RuntimeError("qk_norm_rope_store: query [N, Hq, D] and key [N, Hkv, D] with contiguous heads")
    if key.dtype != query.dtype or q_weight.dtype != query.dtype or k_weight.dtype != query.dtype:
        raise RuntimeError("qk_norm_rope_store: query, key and both weights must share one dtype")
    if q_weight.numel() != d or k_weight.numel() != d or not (q_weight.is_contiguous() and k_weight.is_contiguous()):
        raise RuntimeError("qk_norm_rope_store: weights must be contiguous [head_dim]")
    if positions.dtype != torch.int64 or positions.numel() != n:
        raise RuntimeError("qk_norm_rope_store: positions must be int64 [N]")
    if cos_sin_cache.dtype != torch.float32 or not cos_sin_cache.is_contiguous():
        raise RuntimeError("qk_norm_rope_store: cos_sin_cache must be contiguous float32")
    max_pos = cos_sin_cache.shape[0]
    if cos_sin_cache.numel() != max_pos * rotary_dim:
        raise RuntimeError("qk_norm_rope_store: cos_sin_cache must be [max_position, rotary_dim]")
    store = k_cache is not None and k_cache.numel() > 0 and v_cache is not None and v_cache.numel() > 0
    fp8 = store and k_cache.dtype == torch.float8_e4m3fn
    if store:
        if value is None or value.shape != key.shape or value.stride(-1) != 1 or value.stride(1) != d:
            raise RuntimeError("qk_norm_rope_store: value must be [N, Hkv, D] with contiguous heads")
        if slot_mapping is None or slot_mapping.dtype != torch.int32 or slot_mapping.numel() != n:
            raise RuntimeError("qk_norm_rope_store: slot_mapping must be int32 [N]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise RuntimeError("qk_norm_rope_store: caches must be contiguous")
        if fp8 and (k_scale is None or v_scale is None):
            raise RuntimeError("qk_norm_rope_store: an fp8 cache needs k_scale and v_scale")
        if not fp8 and k_cache.dtype != key.dtype:
            raise RuntimeError(f"qk_norm_rope_store: cache dtype {k_cache.dtype} != key dtype {key.dtype}")
    if q_out is None:
        q_out = torch.empty(n, hq, d, dtype=query.dtype, device=query.device)
    if k_out is None:
        k_out = torch.empty(n, hkv, d, dtype=key.dtype, device=key.device)
    if q_out.shape != query.shape or k_out.shape != key.shape or q_out.stride(-1) != 1 or k_out.stride(1) != d:
        raise RuntimeError("qk_norm_rope_store: q_out/k_out shapes must match query/key")
    num_slots = k_cache.numel() // (hkv * d) if store else 0
    args = (
        ptr(query), query.stride(0), query.stride(1), ptr(key), key.stride(0),
        ptr(value) if store else None, value.stride(0) if store else 0, ptr(positions), ptr(cos_sin_cache),
        max_pos, int(rotary_dim), ptr(q_weight), ptr(k_weight), float(eps), float(weight_offset),
        ptr(q_out), q_out.stride(0), q_out.stride(1), ptr(k_out), k_out.stride(0),
        ptr(k_cache) if store else None, ptr(v_cache) if store else None,
        ptr(slot_mapping) if store else None, num_slots, n, hq, hkv, d, dtype_code(query.dtype),
        dtype_code(k_cache.dtype) if store else dtype_code(query.dtype),
        ptr(k_scale) if fp8 else None, ptr(v_scale) if fp8 else None, stream_of(query))
    if _return_args:
        return args
    check(lib().nq_qk_norm_rope_store(*args), "qk_norm_rope_store")
    return q_out, k_out


def gdn_decode(query, key, value, a, b, A_log, dt_bias, state, state_indices, out=None):
    """Gated DeltaNet decode step for a batch; ``state`` is updated in place.

    Replaces ``decode_gated_delta_rule`` (layers/gated_delta_net.py:85-122)
    and the state slot's read/write around it, for all sequences at once:
    ``query/key [B, H, K]`` (or ``[B, 1, H, K]``), ``value [B, HV, V]``,
    ``a/b [B, HV]``, ``A_log/dt_bias [HV]`` (float32), ``state`` the float32
    pool ``[num_slots, HV, V, K]`` and ``state_indices [B]`` int32 (slots
    outside the pool skip their sequence).  Key heads map to value heads as
    ``h = hv // (HV // H)`` (the reference's repeat_interleave).  Returns
    ``out [B, HV, V]``.
    """
    require_cuda(query, key, value, a, b, A_log, dt_bias, state, state_indices, what="gdn_decode")
    q3 = query.reshape(query.shape[0], -1, query.shape[-1]) if query.dim() == 4 else query
    k3 = key.reshape(key.shape[0], -1, key.shape[-1]) if key.dim() == 4 else key
    v3 = value.reshape(value.shape[0], -1, value.shape[-1]) if value.dim() == 4 else value
    B, H, K = q3.shape
    _, HV, V = v3.shape
    for t, what in ((q3, "query"), (k3, "key"), (v3, "value")):
        if t.stride(-1) != 1 or t.stride(1) != t.shape[-1] or t.dtype != q3.dtype:
            raise RuntimeError(f"gdn_decode: {what} must be [B, heads, dim] contiguous over (head, dim)")
    a2, b2 = a.reshape(B, HV), b.reshape(B, HV)
    if a2.stride(-1) != 1 or b2.stride(-1) != 1 or a2.dtype != q3.dtype or b2.dtype != q3.dtype:
        raise RuntimeError("gdn_decode: a and b must be [B, HV] rows of the query's dtype")
    if A_log.dtype != torch.float32 or dt_bias.dtype != torch.float32:
        raise RuntimeError("gdn_decode: A_log and dt_bias must be float32")
    if state.dtype != torch.float32 or not state.is_contiguous() or state.shape[1:] != (HV, V, K):
        raise RuntimeError("gdn_decode: state must be a contiguous float32 pool [slots, HV, V, K]")
    if state_indices.dtype != torch.int32 or state_indices.numel() != B:
        raise RuntimeError("gdn_decode: state_indices must be int32 [B]")
    if out is None:
        out = torch.empty(B, HV, V, dtype=q3.dtype, device=q3.device)
    rc = lib().nq_gdn_decode(ptr(q3), q3.stride(0), ptr(k3), k3.stride(0), ptr(v3), v3.stride(0), ptr(a2),
                             a2.stride(0), ptr(b2), b2.stride(0), ptr(A_log.contiguous()),
                             ptr(dt_bias.contiguous()), ptr(state), ptr(state_indices), state.shape[0],
                             ptr(out), out.stride(0), B, H, HV, K, V, dtype_code(q3.dtype), stream_of(q3))
    check(rc, "gdn_decode")
    return out


def _overlaps(x, y):
    """Whether the memory spans of two tensors intersect."""
    def span(t):
        lo = t.data_ptr()
        n = sum((d - 1) * st for d, st in zip(t.shape, t.stride())) + 1 if t.numel() else 0
        return lo, lo + n * t.element_size()
    (a0, a1), (b0, b1) = span(x), span(y)
    return a0 < b1 and b0 < a1


def gdn_prefill(query, key, value, a, b, A_log, dt_bias, cu_seqlens, state, state_indices,
                initial_state_from_slot=False, out=None):
    """Gated DeltaNet prefill for packed sequences; final states go to the pool.

    Replaces ``chunk_gated_delta_rule`` (layers/gated_delta_net.py:44-82) with
    the gating before it and the pool write after it, for every sequence of
    the batch at once: ``query/key [T, H, K]``, ``value [T, HV, V]``,
    ``a/b [T, HV]`` packed by ``cu_seqlens [N + 1]`` int32; ``state`` the
    float32 pool and ``state_indices [N]`` int32.  Returns ``out [T, HV, V]``.
    """
    require_cuda(query, key, value, a, b, A_log, dt_bias, cu_seqlens, state, state_indices, what="gdn_prefill")
    T_, H, K = query.shape
    HV, V = value.shape[1], value.shape[2]
    for t, what in ((query, "query"), (key, "key"), (value, "value")):
        if t.stride(-1) != 1 or t.stride(1) != t.shape[-1] or t.dtype != query.dtype or t.shape[0] != T_:
            raise RuntimeError(f"gdn_prefill: {what} must be [T, heads, dim] contiguous over (head, dim)")
    a2, b2 = a.reshape(T_, HV), b.reshape(T_, HV)
    if a2.stride(-1) != 1 or b2.stride(-1) != 1 or a2.dtype != query.dtype or b2.dtype != query.dtype:
        raise RuntimeError("gdn_prefill: a and b must be [T, HV] rows of the query's dtype")
    if A_log.dtype != torch.float32 or dt_bias.dtype != torch.float32:
        raise RuntimeError("gdn_prefill: A_log and dt_bias must be float32")
    if state.dtype != torch.float32 or not state.is_contiguous() or state.shape[1:] != (HV, V, K):
        raise RuntimeError("gdn_prefill: state must be a contiguous float32 pool [slots, HV, V, K]")
    n = cu_seqlens.numel() - 1
    if cu_seqlens.dtype != torch.int32 or state_indices.dtype != torch.int32 or state_indices.numel() != n:
        raise RuntimeError("gdn_prefill: cu_seqlens [N+1] and state_indices [N] must be int32")
    if out is None:
        out = torch.empty(T_, HV, V, dtype=query.dtype, device=query.device)
    # the kernel keeps each token's gates in its output rows before writing
    # the output there, so out may not share memory with an input
    for t, what in ((query, "query"), (key, "key"), (value, "value"), (a2, "a"), (b2, "b")):
        if _overlaps(out, t):
            raise RuntimeError(f"gdn_prefill: out must not overlap {what}")
    rc = lib().nq_gdn_prefill(ptr(query), query.stride(0), ptr(key), key.stride(0), ptr(value), value.stride(0),
                              ptr(a2), a2.stride(0), ptr(b2), b2.stride(0), ptr(A_log.contiguous()),
                              ptr(dt_bias.contiguous()), ptr(cu_seqlens), n, ptr(state), ptr(state_indices),
                              state.shape[0], 1 if initial_state_from_slot else 0, ptr(out), out.stride(0),
                              H, HV, K, V, dtype_code(query.dtype), stream_of(query))
    check(rc, "gdn_prefill")
    return out


def gated_rmsnorm(x, gate, weight, eps, out=None):
    """``RMSNormGated(x, gate)`` (layers/layernorm.py:143-157) in one pass over
    rows of the last dimension: ``x, gate [..., D]`` (16-bit, same dtype),
    ``weight [D]`` float32.  ``out=x`` normalizes in place."""
    require_cuda(x, gate, weight, out, what="gated_rmsnorm")
    d = x.shape[-1]
    x2, g2 = x.reshape(-1, d), gate.reshape(-1, d)
    if x2.stride(-1) != 1 or g2.stride(-1) != 1 or gate.dtype != x.dtype or g2.shape[0] != x2.shape[0]:
        raise RuntimeError("gated_rmsnorm: x and gate must be [..., D] rows of one dtype")
    if weight.dtype != torch.float32 or weight.numel() != d or not weight.is_contiguous():
        raise RuntimeError("gated_rmsnorm: weight must be contiguous float32 [D]")
    if out is None:
        out = torch.empty_like(x)
    o2 = out.reshape(-1, d)
    check(lib().nq_gated_rmsnorm(ptr(x2), x2.stride(0), ptr(g2), g2.stride(0), ptr(weight), float(eps), ptr(o2),
                                 o2.stride(0), x2.shape[0], d, dtype_code(x.dtype), stream_of(x)), "gated_rmsnorm")
    return out


def gdn_conv1d(x, weight, conv_state, state_indices, cu_seqlens=None, out=None):
    """Causal depthwise conv1d + silu with the conv state pool (GatedDeltaNet,
    layers/gated_delta_net.py:178-180, 207-213, 218-227).

    ``x [rows, C]`` 16-bit; ``weight [C, K]`` (or ``[C, 1, K]``);
    ``conv_state [slots, C, K - 1]`` of x's dtype; ``state_indices [N]``
    int32.  Without ``cu_seqlens`` (decode) row b is sequence b's new token;
    with it (prefill) the rows are packed sequences starting from zero.
    Returns ``out [rows, C]``; the slots are updated in place.
    """
    require_cuda(x, weight, conv_state, state_indices, cu_seqlens, what="gdn_conv1d")
    rows, C = x.shape
    w2 = weight.reshape(C, -1)
    K = w2.shape[1]
    if x.stride(-1) != 1 or not w2.is_contiguous() or w2.dtype != x.dtype:
        raise RuntimeError("gdn_conv1d: x rows contiguous; weight contiguous [C, K] of x's dtype")
    if conv_state.dtype != x.dtype or not conv_state.is_contiguous() or conv_state.shape[1:] != (C, K - 1):
        raise RuntimeError("gdn_conv1d: conv_state must be contiguous [slots, C, K - 1] of x's dtype")
    n = rows if cu_seqlens is None else cu_seqlens.numel() - 1
    if state_indices.dtype != torch.int32 or state_indices.numel() != n:
        raise RuntimeError("gdn_conv1d: state_indices must be int32 [N]")
    if cu_seqlens is not None and cu_seqlens.dtype != torch.int32:
        raise RuntimeError("gdn_conv1d: cu_seqlens must be int32")
    if out is None:
        out = torch.empty_like(x)
    check(lib().nq_gdn_conv1d(ptr(x), x.stride(0), ptr(w2), K, ptr(cu_seqlens), n, ptr(conv_state),
                              ptr(state_indices), conv_state.shape[0], 0, ptr(out), out.stride(0), C,
                              dtype_code(x.dtype), stream_of(x)), "gdn_conv1d")
    return out


__all__ = ["store_kvcache", "paged_decode", "varlen_prefill", "prepare_decode", "decode_plan", "qk_norm_rope_store",
           "output_gate", "gdn_decode", "gdn_prefill", "gated_rmsnorm", "gdn_conv1d",
           "decode_workspace", "prefill_workspace", "release_workspaces", "decode_schedule", "_lib"]
