"""Attention-metadata half of the reference's ``ModelRunner``.

Restates, for the paged attention path only, engine/model_runner.py:
``allocate_kv_cache`` (:186-204), ``allocate_decode_buffers`` (:206-218),
``prepare_block_tables`` (:236-240), ``prepare_prefill`` (:242-283) and
``prepare_decode`` (:285-306), ``run_model`` (:319-336) and
``capture_cudagraph`` (:421-456).  The decode metadata kernel is the HIP
``nq_prepare_decode`` instead of Triton.  Model construction, sampling,
TP control plane and the engine loop are out of scope: the caller hands
``capture_cudagraph`` the model (anything called as
``model(input_ids, positions)`` whose attention layers read ``get_context()``).

fp8 extension: ``allocate_kv_cache(..., kv_cache_dtype=torch.float8_e4m3fn)``
also creates ``kv_scales [2, L, Hkv]`` float32 (initialised to 1) and binds
``module.k_scale = kv_scales[0, l]`` / ``module.v_scale = kv_scales[1, l]``;
``calibrate_kv_scales`` sets them to absmax/448 per (layer, kv head).  The
pool is sized from the memory budget with the *cache* dtype's item size, so
an fp8 pool holds twice the blocks of a bf16 one in the same budget.
"""
from __future__ import annotations

import torch

from .. import kernels
from ..utils.context import get_context, reset_context, set_context


class ModelRunner:

    def __init__(self, block_size: int = 256, max_num_seqs: int = 512, device="cuda", config=None):
        """``config``, when given, is an object with the reference Config's
        fields (config/config.py:6-24) that ``allocate_kv_cache()`` reads:
        ``hf_config`` (``num_hidden_layers``, ``num_key_value_heads``,
        ``head_dim`` or ``hidden_size`` / ``num_attention_heads``, ``dtype``),
        ``gpu_memory_utilization``, ``kvcache_block_size``, ``max_num_seqs``,
        ``num_kvcache_blocks`` (set here) and optionally
        ``tensor_parallel_size`` and ``kv_cache_dtype`` (the fp8 extension).
        Its block size and sequence count then take precedence."""
        if config is not None:
            block_size = config.kvcache_block_size
            max_num_seqs = config.max_num_seqs
        self.config = config
        self.world_size = getattr(config, "tensor_parallel_size", 1) if config is not None else 1
        self.block_size = block_size
        self.max_num_seqs = max_num_seqs
        self.device = torch.device(device)
        self._pin = self.device.type == "cuda"
        self.kv_cache = None
        self.kv_scales = None
        self.model = None
        self.enforce_eager = False
        self.graphs = {}
        self.graph_bs = []
        self.graph_pool = None
        self.graph_vars = None
        # MRV2-style persistent batch: batch_idx -> request slot, and the last
        # sampled token of every slot (engine/model_runner.py:100-106).
        self.sampled_token_ids_gpu = torch.zeros(max_num_seqs, dtype=torch.int64, device=self.device)
        self.batch_slots_gpu = torch.arange(max_num_seqs, dtype=torch.int64, device=self.device)
        self.allocate_decode_buffers()

    # ------------------------------------------------------------- KV pool
    def kv_block_bytes(self, num_layers: int, num_kv_heads: int, head_dim: int, kv_dtype: torch.dtype) -> int:
        """Bytes of one block of every layer's K and V
        (engine/model_runner.py:195), with the cache dtype's item size."""
        item = torch.empty((), dtype=kv_dtype).element_size()
        return 2 * num_layers * self.block_size * num_kv_heads * head_dim * item

    def budget_blocks(self, block_bytes: int, gpu_memory_utilization: float, mem_info=None, stats=None) -> int:
        """Blocks that fit the memory budget (engine/model_runner.py:189-196):
        ``(total * utilization - used - peak + current) // block_bytes``, with
        ``free, total = mem_get_info()``, ``used = total - free`` and the
        allocator's peak and current allocated bytes (the peak of the warm-up
        run is reserved for activations).  ``mem_info`` / ``stats`` stand in
        for the device queries."""
        free, total = mem_info if mem_info is not None else torch.cuda.mem_get_info(self.device)
        used = total - free
        st = stats if stats is not None else torch.cuda.memory_stats(self.device)
        peak = st["allocated_bytes.all.peak"]
        current = st["allocated_bytes.all.current"]
        return int(total * gpu_memory_utilization - used - peak + current) // block_bytes

    def allocate_kv_cache(self, model=None, num_layers: int | None = None, num_blocks: int | None = None,
                          num_kv_heads: int | None = None, head_dim: int | None = None,
                          dtype: torch.dtype | None = None, kv_cache_dtype: torch.dtype | None = None,
                          gpu_memory_utilization: float | None = None):
        """One tensor ``[2, L, num_blocks, block_size, Hkv, D]`` and per-layer
        views bound to every module with ``k_cache``/``v_cache`` attributes
        (engine/model_runner.py:186-204).

        Called as the reference calls it, ``allocate_kv_cache()``, every
        argument comes from ``self.config`` and ``self.model``, and the block
        count from the memory budget (``budget_blocks``), which it also
        stores in ``config.num_kvcache_blocks``.  Explicit arguments override
        those; ``num_blocks=None`` sizes from the budget
        (``gpu_memory_utilization``, default the config's or 0.9).  Returns
        the number of layers bound."""
        cfg = self.config
        hf = getattr(cfg, "hf_config", None)
        model = model if model is not None else self.model
        if model is None:
            raise ValueError("allocate_kv_cache: no model (pass one, or set runner.model)")
        if hf is not None:
            num_layers = num_layers if num_layers is not None else hf.num_hidden_layers
            num_kv_heads = num_kv_heads if num_kv_heads is not None else hf.num_key_value_heads // self.world_size
            if head_dim is None:
                head_dim = getattr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
            dtype = dtype if dtype is not None else hf.dtype
            kv_cache_dtype = kv_cache_dtype if kv_cache_dtype is not None else getattr(cfg, "kv_cache_dtype", None)
        if None in (num_layers, num_kv_heads, head_dim, dtype):
            raise ValueError("allocate_kv_cache: layers, kv heads, head_dim and dtype are needed "
                             "(as arguments or from config.hf_config)")
        kv_dtype = kv_cache_dtype or dtype
        if num_blocks is None:
            util = gpu_memory_utilization if gpu_memory_utilization is not None else \
                getattr(cfg, "gpu_memory_utilization", 0.9)
            num_blocks = self.budget_blocks(self.kv_block_bytes(num_layers, num_kv_heads, head_dim, kv_dtype), util)
            assert num_blocks > 0, "allocate_kv_cache: the memory budget holds no KV block"
        if cfg is not None:
            cfg.num_kvcache_blocks = num_blocks
        self.model = model
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

    def calibrate_kv_scales(self, kv_per_layer):
        """fp8 pools: ``kv_scales[0, l, h] = absmax(K_l[..., h, :]) / 448``
        and likewise for V, so the largest calibration value of each
        (layer, kv head) maps to e4m3's largest finite value and nothing
        saturates.  ``kv_per_layer[l] = (k, v)``, each a tensor ``[..., Hkv,
        D]`` or a list of them (e.g. the new keys and values of a
        calibration prefill, and the prefix already in the pool).  A head
        whose values are all zero keeps scale 1.  The scales are updated in
        place, so the layers' bound ``k_scale`` / ``v_scale`` views see them.

        The reference allocates the pool here (engine/model_runner.py:186-204)
        but has no fp8 cache; the rule is the one its fp8 KV configuration
        states (per-(layer, kv_head) absmax/448)."""
        if self.kv_scales is None:
            raise RuntimeError("calibrate_kv_scales: the KV pool is not float8_e4m3fn")
        _, n_layers, hkv = self.kv_scales.shape
        if len(kv_per_layer) != n_layers:
            raise ValueError(f"calibrate_kv_scales: {len(kv_per_layer)} layers given, the pool has {n_layers}")
        for layer, pair in enumerate(kv_per_layer):
            for which, xs in enumerate(pair):
                amax = None
                for x in (xs if isinstance(xs, (list, tuple)) else [xs]):
                    if x.shape[-2] != hkv:
                        raise ValueError(f"calibrate_kv_scales: {x.shape[-2]} kv heads, the pool has {hkv}")
                    a = x.float().abs().reshape(-1, hkv, x.shape[-1]).amax(dim=(0, 2))
                    amax = a if amax is None else torch.maximum(amax, a)
                s = (amax / 448.0).to(self.kv_scales.device)
                self.kv_scales[which, layer] = torch.where(s > 0, s, torch.ones_like(s))
        return self.kv_scales

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
        input_ids = self._to_device(input_ids, torch.int64)
        positions = self._to_device(positions, torch.int64)
        cu_seqlens_q = self._to_device(cu_seqlens_q, torch.int32)
        cu_seqlens_k = self._to_device(cu_seqlens_k, torch.int32)
        slot_mapping = self._to_device(slot_mapping, torch.int32)
        set_context(True, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping, None,
                    block_tables)
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

    # ------------------------------------------------------- graph capture
    @torch.inference_mode()
    def run_model(self, input_ids: torch.Tensor, positions: torch.Tensor, is_prefill: bool):
        """engine/model_runner.py:319-336: prefill, eager mode and batches
        above 512 run the model directly; a decode batch replays the graph of
        the smallest bucket that holds it, after copying its inputs into the
        static ``graph_vars`` -- padding rows get ``slot_mapping = -1`` (the
        store skips them) and ``context_lens = 0`` (decode writes zeros), and
        block-table entries past a row's context are never read.  Returns the
        model's ``compute_logits`` of the output when it has one, else the
        output (``[bs, hidden]``)."""
        model = self.model
        if is_prefill or self.enforce_eager or input_ids.size(0) > 512 or not self.graphs:
            return self._logits(model(input_ids, positions))
        bs = input_ids.size(0)
        context = get_context()
        graph = self.graphs[next(x for x in self.graph_bs if x >= bs)]
        gv = self.graph_vars
        gv["input_ids"][:bs] = input_ids
        gv["positions"][:bs] = positions
        gv["slot_mapping"].fill_(-1)
        gv["slot_mapping"][:bs] = context.slot_mapping
        gv["context_lens"].zero_()
        gv["context_lens"][:bs] = context.context_lens
        gv["block_tables"][:bs, :context.block_tables.size(1)] = context.block_tables
        graph.replay()
        return self._logits(gv["outputs"][:bs])

    def _logits(self, hidden):
        f = getattr(self.model, "compute_logits", None)
        return f(hidden) if f is not None else hidden

    @torch.inference_mode()
    def capture_cudagraph(self, model, hidden_size: int, max_model_len: int,
                          dtype: torch.dtype | None = None):
        """engine/model_runner.py:421-456: one HIP graph per decode batch
        bucket ``[1, 2, 4, 8, 16, 32, ..]`` up to ``min(max_num_seqs, 512)``,
        largest first, all in one memory pool, over static ``graph_vars``
        sized for the largest bucket and ``max_model_len``'s block-table
        width.

        Differences from the reference, both so a capture cannot disturb the
        cache or leave a batch size without a graph: the capture inputs have
        ``slot_mapping = -1`` (the reference's zeros make the warmup and
        capture store into slot 0), and when ``max_bs`` is not itself a
        bucket it is added as the last one (the reference's bucket list skips
        sizes between its last multiple of 16 and ``max_bs``, or names
        buckets above ``max_bs`` that capture fewer rows).

        Every kernel the decode step launches keeps its buffers across
        replays: the split-K workspace belongs to the capture stream and is
        never freed while a graph may hold it (a later, larger plan on that
        stream allocates a new one and keeps the old alive), and nothing in
        the step records a memset node.
        """
        self.model = model
        dev = self.device
        max_bs = min(self.max_num_seqs, 512)
        max_num_blocks = (max_model_len + self.block_size - 1) // self.block_size
        input_ids = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        positions = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        slot_mapping = torch.full((max_bs,), -1, dtype=torch.int32, device=dev)
        context_lens = torch.zeros(max_bs, dtype=torch.int32, device=dev)
        block_tables = torch.zeros(max_bs, max_num_blocks, dtype=torch.int32, device=dev)
        outputs = torch.zeros(max_bs, hidden_size, dtype=dtype or torch.get_default_dtype(), device=dev)
        self.graph_bs = [x for x in [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) if x <= max_bs]
        if self.graph_bs[-1] != max_bs:
            self.graph_bs.append(max_bs)
        self.graphs = {}
        self.graph_pool = None
        for bs in reversed(self.graph_bs):
            graph = torch.cuda.CUDAGraph()
            set_context(False, slot_mapping=slot_mapping[:bs], context_lens=context_lens[:bs],
                        block_tables=block_tables[:bs])
            outputs[:bs] = model(input_ids[:bs], positions[:bs])    # warmup
            with torch.cuda.graph(graph, self.graph_pool):
                outputs[:bs] = model(input_ids[:bs], positions[:bs])    # capture
            if self.graph_pool is None:
                self.graph_pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
            reset_context()
        self.graph_vars = dict(input_ids=input_ids, positions=positions, slot_mapping=slot_mapping,
                               context_lens=context_lens, block_tables=block_tables, outputs=outputs)
