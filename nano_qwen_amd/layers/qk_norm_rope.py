"""Fused q/k Gemma RMS norm + rotary embedding + KV store for Qwen3.5 attention.

Drop-in for the three calls of ``Qwen3_5Attention.forward`` that sit between
the projections and the attention call (models/qwen3_5.py:135-137)::

    query = self.q_norm(query)
    key = self.k_norm(key)
    query, key = self.rotary_emb(positions, query, key)
    attn_output = self.attn(query, key, value)

becomes::

    query, key = qk_norm_rope_store(positions, query, key, value,
                                    self.q_norm, self.k_norm, self.rotary_emb, self.attn)
    attn_output = self.attn(query, key, value, kv_stored=True)

The modules are the reference's own (``GemmaRMSNorm``: ``.weight``, ``.eps``,
layers/layernorm.py; ``InterleavedMRoPE`` / ``RotaryEmbedding``:
``.cos_sin_cache`` ``[max_position, 1, R]`` float32, layers/rotary_embedding.py);
only their parameters and buffers are read.  The KV store that
``Attention.forward`` would make (layers/attention.py:62-63) happens inside the
same launch, into ``attn``'s caches at the current context's slots, and is
skipped while the caches are empty (warmup), as there.
"""
from __future__ import annotations

import torch

from .. import kernels
from ..utils.context import get_context


def qk_norm_rope_store(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                       value: torch.Tensor, q_norm, k_norm, rotary_emb, attn=None,
                       weight_offset: float = 1.0):
    """Returns ``(query, key)`` normalized and rotated; stores key/value rows.

    ``query [N, Hq, D]`` may be the strided query half of ``q_proj``'s output.
    ``weight_offset`` is 1.0 for the Gemma norm (``x * (1 + w)``) and 0.0 for a
    plain RMSNorm (``x * w``).
    """
    if q_norm.eps != k_norm.eps:
        raise RuntimeError("qk_norm_rope_store: q_norm and k_norm must share eps")
    table = rotary_emb.cos_sin_cache
    rot = int(getattr(rotary_emb, "rotary_dim", table.shape[-1]))
    k_cache = v_cache = slots = k_scale = v_scale = None
    if attn is not None and attn.k_cache.numel() and attn.v_cache.numel():
        k_cache, v_cache = attn.k_cache, attn.v_cache
        slots = get_context().slot_mapping
        k_scale, v_scale = attn.k_scale, attn.v_scale
    return kernels.qk_norm_rope_store(positions, query, key, value, q_norm.weight.detach(),
                                      k_norm.weight.detach(), q_norm.eps, table, rot,
                                      k_cache=k_cache, v_cache=v_cache, slot_mapping=slots,
                                      k_scale=k_scale, v_scale=v_scale, weight_offset=weight_offset)
