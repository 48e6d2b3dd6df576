"""Drop-in ``Attention`` layer and ``store_kvcache`` on the HIP kernels.

Same constructor, attributes and ``forward(q, k, v)`` contract as the
reference's layers/attention.py:33-75; the Triton scatter and the flash_attn
calls are replaced by the gfx950 kernels of ``libnq_attn.so``.

fp8 extension (absent from the reference): when the runner binds
``float8_e4m3fn`` caches it also binds ``k_scale`` / ``v_scale`` (float32
``[Hkv]``, one scale per kv head of this layer); the store quantizes with
them and both attention kernels dequantize in registers.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import kernels
from ..utils.context import get_context


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor, k_scale: torch.Tensor | None = None,
                  v_scale: torch.Tensor | None = None):
    """layers/attention.py:33-40, same asserts, then the HIP scatter."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    kernels.store_kvcache(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale)


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = self.v_scale = None

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_stored: bool = False,
                gate: torch.Tensor | None = None):
        """layers/attention.py:59-75: store, then prefill or paged decode
        (in decode the store and the attention are one launch).

        ``kv_stored=True`` skips the store because the caller already made it
        (``layers.qk_norm_rope_store`` stores in the same launch as the q/k
        norm and rotation).  ``gate [N, Hq, D]`` returns
        ``o * sigmoid(gate)``, Qwen3.5's output gate (models/qwen3_5.py:140-142):
        inside the decode kernel's store, or one in-place pass after prefill.
        """
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        store = k_cache.numel() and v_cache.numel() and not kv_stored
        if store and not context.is_prefill:
            # decode: the store rides in the decode launch (nq_paged_decode_store);
            # the reference's asserts of the store still apply
            N, num_heads, head_dim = k.shape
            assert k.stride(-1) == 1 and v.stride(-1) == 1
            assert k.stride(1) == head_dim and v.stride(1) == head_dim
            assert k_cache.stride(1) == num_heads * head_dim and v_cache.stride(1) == num_heads * head_dim
            assert context.slot_mapping.numel() == N
            return kernels.paged_decode(q.unsqueeze(1), k_cache, v_cache,
                                        cache_seqlens=context.context_lens,
                                        block_table=context.block_tables, softmax_scale=self.scale,
                                        k_scale=self.k_scale, v_scale=self.v_scale,
                                        gate=None if gate is None else gate.unsqueeze(1),
                                        k=k, v=v, slot_mapping=context.slot_mapping)
        if store:
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping, self.k_scale, self.v_scale)
        if context.is_prefill:
            k_scale = v_scale = None
            if context.block_tables is not None:    # prefix cache
                k, v = k_cache, v_cache
                k_scale, v_scale = self.k_scale, self.v_scale
            o = kernels.varlen_prefill(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k,
                                       context.max_seqlen_q, context.max_seqlen_k,
                                       softmax_scale=self.scale, causal=True,
                                       block_table=context.block_tables,
                                       k_scale=k_scale, v_scale=v_scale, gate=gate)
        else:    # decode
            o = kernels.paged_decode(q.unsqueeze(1), k_cache, v_cache,
                                     cache_seqlens=context.context_lens,
                                     block_table=context.block_tables, softmax_scale=self.scale,
                                     k_scale=self.k_scale, v_scale=self.v_scale,
                                     gate=None if gate is None else gate.unsqueeze(1))
        return o
