"""Attention-metadata half of the reference's ``ModelRunner``.

Restates, for the paged attention path only, engine/model_runner.py:
``allocate_kv_cache`` (:186-204), ``allocate_decode_buffers`` (:206-218),
``prepare_block_tables`` (:236-240), ``prepare_prefill`` (:242-283) and
``prepare_decode`` (:285-306).  The decode metadata kernel is the HIP
``nq_prepare_decode`` instead of Triton.  Model construction, sampling,
TP control plane and the engine loop are out of scope.

fp8 extension: ``allocate_kv_cache(..., kv_cache_dtype=torch.float8_e4m3fn)``
also creates ``kv_scales [2, L, Hkv]`` float32 (initialised to 1) and binds
``module.k_scale = kv_scales[0, l]`` / ``module.v_scale = kv_scales[1, l]``.
"""
from __future__ import annotations

import torch

from .. import kernels
from ..utils.context import set_context


class ModelRunner:

    def __init__(self, block_size: int = 256, max_num_seqs: int = 512, device="cuda"):
        self.block_size = block_size
        self.max_num_seqs = max_num_seqs
        self.device = torch.device(device)
        self._pin = self.device.type == "cuda"
        self.kv_cache = None
        self.kv_scales = None
        # MRV2-style persistent batch: batch_idx -> request slot, and the last
        # sampled token of every slot (engine/model_runner.py:100-106).
        self.sampled_token_ids_gpu = torch.zeros(max_num_seqs, dtype=torch.int64, device=self.device)
        self.batch_slots_gpu = torch.arange(max_num_seqs, dtype=torch.int64, device=self.device)
        self.allocate_decode_buffers()

    # ------------------------------------------------------------- KV pool
    def allocate_kv_cache(self, model, num_layers: int, num_blocks: int, num_kv_heads: int,
                          head_dim: int, dtype: torch.dtype, kv_cache_dtype: torch.dtype | None = None):
        """One tensor ``[2, L, num_blocks, block_size, Hkv, D]`` and per-layer
        views bound to every module with ``k_cache``/``v_cache`` attributes
        (engine/model_runner.py:198-204)."""
        kv_dtype = kv_cache_dtype or dtype
        self.kv_cache = torch.empty(2, num_layers, num_blocks, self.block_size, num_kv_heads, head_dim,
                                    dtype=kv_dtype, device=self.device)
        if kv_dtype == torch.float8_e4m3fn:
            self.kv_scales = torch.ones(2, num_layers, num_kv_heads, dtype=torch.float32,
                                        device=self.device)
        modules = model.modules() if hasattr(model, "modules") else model
        layer_id = 0
        for module in modules:
            if hasattr(module, "k_cache") and hasattr(module, "v_cache"):
                module.k_cache = self.kv_cache[0, layer_id]
                module.v_cache = self.kv_cache[1, layer_id]
                if self.kv_scales is not None:
                    module.k_scale = self.kv_scales[0, layer_id]
                    module.v_scale = self.kv_scales[1, layer_id]
                layer_id += 1
        return layer_id

    def allocate_decode_buffers(self):
        size = self.max_num_seqs
        self.decode_cpu = {
            "seq_lens": torch.empty(size, dtype=torch.int32, pin_memory=self._pin),
            "last_block_ids": torch.empty(size, dtype=torch.int32, pin_memory=self._pin),
        }
        self.decode_gpu = {name: torch.empty_like(t, device=self.device) for name, t in self.decode_cpu.items()}
        self.decode_gpu.update({
            "input_ids": torch.empty(size, dtype=torch.int64, device=self.device),
            "positions": torch.empty(size, dtype=torch.int64, device=self.device),
            "slot_mapping": torch.empty(size, dtype=torch.int32, device=self.device),
            "context_lens": torch.empty(size, dtype=torch.int32, device=self.device),
        })

    # ------------------------------------------------------------- metadata
    def _to_device(self, data, dtype):
        t = torch.tensor(data, dtype=dtype, pin_memory=self._pin)
        return t.to(self.device, non_blocking=True)

    def prepare_block_tables(self, seqs):
        max_len = max(len(seq.block_table) for seq in seqs)
        block_tables = [seq.block_table + [-1] * (max_len - len(seq.block_table)) for seq in seqs]
        return self._to_device(block_tables, torch.int32)

    def prepare_prefill(self, seqs):
        """engine/model_runner.py:242-283."""
        input_ids, positions, slot_mapping = [], [], []
        cu_seqlens_q, cu_seqlens_k = [0], [0]
        max_seqlen_q = max_seqlen_k = 0
        block_tables = None
        bs = self.block_size
        for seq in seqs:
            start = seq.num_cached_tokens
            seqlen_q = seq.num_scheduled_tokens
            end = start + seqlen_q
            seqlen_k = end
            input_ids.extend(seq[start:end])
            positions.extend(range(start, end))
            cu_seqlens_q.append(cu_seqlens_q[-1] + seqlen_q)
            cu_seqlens_k.append(cu_seqlens_k[-1] + seqlen_k)
            max_seqlen_q = max(seqlen_q, max_seqlen_q)
            max_seqlen_k = max(seqlen_k, max_seqlen_k)
            if not seq.block_table:    # warmup
                continue
            start_block = start // bs
            end_block = (end + bs - 1) // bs
            for i in range(start_block, end_block):
                base = seq.block_table[i] * bs
                lo = start % bs if i == start_block else 0
                hi = end - i * bs if i == end_block - 1 else bs
                slot_mapping.extend(range(base + lo, base + hi))
        if cu_seqlens_k[-1] > cu_seqlens_q[-1]:    # prefix cache
            block_tables = self.prepare_block_tables(seqs)
        total_k = cu_seqlens_k[-1]
        input_ids = self._to_device(input_ids, torch.int64)
        positions = self._to_device(positions, torch.int64)
        cu_seqlens_q = self._to_device(cu_seqlens_q, torch.int32)
        cu_seqlens_k = self._to_device(cu_seqlens_k, torch.int32)
        slot_mapping = self._to_device(slot_mapping, torch.int32)
        set_context(True, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping, None,
                    block_tables, total_k=total_k)
        return input_ids, positions

    def prepare_decode(self, seqs):
        """engine/model_runner.py:285-306 with the HIP metadata kernel."""
        bs = len(seqs)
        cpu = self.decode_cpu
        for i, seq in enumerate(seqs):
            cpu["seq_lens"][i] = len(seq)
            cpu["last_block_ids"][i] = seq.block_table[-1]
        for name, tensor in cpu.items():
            self.decode_gpu[name][:bs].copy_(tensor[:bs], non_blocking=True)
        gpu = self.decode_gpu
        kernels.prepare_decode(
            self.sampled_token_ids_gpu, self.batch_slots_gpu[:bs], gpu["seq_lens"], gpu["last_block_ids"],
            gpu["input_ids"], gpu["positions"], gpu["context_lens"], gpu["slot_mapping"], bs,
            self.block_size)
        input_ids = gpu["input_ids"][:bs]
        positions = gpu["positions"][:bs]
        slot_mapping = gpu["slot_mapping"][:bs]
        context_lens = gpu["context_lens"][:bs]
        block_tables = self.prepare_block_tables(seqs)
        set_context(False, slot_mapping=slot_mapping, context_lens=context_lens, block_tables=block_tables)
        return input_ids, positions
