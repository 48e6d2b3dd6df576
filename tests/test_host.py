"""Host-side logic and the C ABI surface, on the CPU (no device calls)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import nano_qwen_amd
from nano_qwen_amd import _lib, kernels
from nano_qwen_amd.engine import ModelRunner, Sequence
from nano_qwen_amd.layers import Attention, store_kvcache
from nano_qwen_amd.utils import context as C
from oracle import metadata

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "nq_attn.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(nq_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_header_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert "nq_paged_decode" in names and "nq_varlen_prefill" in names and "nq_store_kvcache" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/nq_attn.h but not exported"
    assert set(names) == set(_lib.EXPORTED), "ctypes signatures out of sync with the header"
    assert lib.nq_abi_version() == 1


def test_abi_rejects_bad_arguments_without_launching():
    lib = _lib.lib()
    # head_dim 64 is not built: NQ_EUNSUPPORTED before any device work
    rc = lib.nq_paged_decode(None, 0, 0, None, None, None, 0, 1, None, None, 0, 0, 2, 8, 2, 64, 256, 1,
                             0.1, 1, 256, None, 0, 2, 2, None, None, None)
    assert rc == -2 and b"head_dim" in lib.nq_last_error()
    rc = lib.nq_paged_decode(None, 0, 0, None, None, None, 0, 1, None, None, 0, 0, 2, 6, 4, 128, 256, 1,
                             0.1, 1, 256, None, 0, 2, 2, None, None, None)
    assert rc == -1  # 6 q heads over 4 kv heads
    rc = lib.nq_store_kvcache(None, 0, None, 0, None, None, None, 3, 10, 8, 128, 2, 2, None, None, None)
    assert rc == -1 and b"null" in lib.nq_last_error()
    assert lib.nq_store_kvcache(None, 0, None, 0, None, None, None, 0, 10, 8, 128, 2, 2, None, None, None) == 0
    rc = lib.nq_varlen_prefill(None, 0, 0, None, None, 0, None, None, 10, 10, None, 0, 0, 0, None, 0, 0, 1, 32, 8,
                               128, 256, 0.1, 1, 2, 1, None, None, None, 0, None)
    assert rc == -2  # bf16 q with f16 kv
    assert lib.nq_prefill_workspace_bytes() >= 36  # 8 per-XCD counters + 1 finish counter
    # a split wider than 63 blocks: each split holds its block-table entries
    # one per lane, so the ABI refuses it (nq_decode_plan never makes one)
    fake = ctypes.c_void_p(1 << 20)
    args = lambda st, ns: (fake, 1024, 128, fake, fake, fake, 64, 64, fake, fake, 1024, 128, 2, 8, 2, 128, 256,
                           64, 0.1, ns, st, fake, 1 << 30, 2, 2, None, None, None)
    rc = lib.nq_paged_decode(*args(63 * 256 // 128 * 128 + 128, 2))
    assert rc == -1 and b"split_tokens" in lib.nq_last_error()
    ns, st = kernels.decode_plan(1, 8, 2, 4096, 256, torch.bfloat16)
    assert st <= 63 * 256
    # the schedule query refuses bad arguments before any device call
    assert lib.nq_decode_schedule(0, 32, 8, 128, 16, 256, 2, 2, 0) == -1
    assert lib.nq_decode_schedule(4, 32, 8, 64, 16, 256, 2, 2, 0) == -2
    # conv1d rows narrower than the channel count overlap: refused
    rc = lib.nq_gdn_conv1d(fake, 512, fake, 4, fake, 2, fake, fake, 4, 0, fake, 1024, 1024, 2, None)
    assert rc == -1 and b"row strides" in lib.nq_last_error()


def test_decode_plan_covers_table_and_respects_env(monkeypatch):
    # A multi-split plan may carry more splits than the table needs: the
    # workspace nq_decode_workspace_bytes sizes from them then also holds the
    # stream-K partials.  With stream-K off the splits cover the table exactly.
    for streamk in ("1", "0"):
        monkeypatch.setenv("NQ_DECODE_STREAMK", streamk)
        for W, B in ((1, 1), (16, 64), (128, 8), (32, 128), (3, 5)):
            ns, st = kernels.decode_plan(B, 32, 8, W, 256, torch.bfloat16)
            cover = -(-W * 256 // st)
            assert st % 128 == 0 and ns * st >= W * 256 and ns >= cover
            assert ns == cover if (streamk == "0" or cover == 1) else True
    monkeypatch.setenv("NQ_DECODE_STREAMK", "0")
    monkeypatch.setenv("NQ_DECODE_SPLIT_TOKENS", "1024")
    ns, st = kernels.decode_plan(8, 64, 8, 128, 256, torch.bfloat16)
    assert (ns, st) == (32, 1024)
    monkeypatch.setenv("NQ_DECODE_STREAMK", "1")
    ns, st = kernels.decode_plan(8, 64, 8, 128, 256, torch.bfloat16)
    assert ns >= 32 and st == 1024
    assert _lib.lib().nq_decode_workspace_bytes(8, 64, 128, 1) == 0
    assert _lib.lib().nq_decode_workspace_bytes(8, 64, 128, 32) >= 8 * 64 * 32 * (128 + 1) * 4


def test_context_roundtrip():
    C.reset_context()
    assert C.get_context().is_prefill is False and C.get_context().block_tables is None
    C.set_context(True, torch.tensor([0, 3]), torch.tensor([0, 5]), 3, 5, torch.tensor([1, 2, 3]))
    ctx = C.get_context()
    assert ctx.is_prefill and ctx.max_seqlen_k == 5 and ctx.context_lens is None
    assert [f for f in C.Context.__slots__] == ["is_prefill", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q",
                                               "max_seqlen_k", "slot_mapping", "context_lens", "block_tables",
                                               "state_indices"]
    C.reset_context()
    assert C.get_context().cu_seqlens_q is None


def test_attention_module_contract():
    a = Attention(32, 128, 128 ** -0.5, 8)
    assert (a.num_heads, a.head_dim, a.num_kv_heads) == (32, 128, 8)
    assert a.k_cache.numel() == 0 and a.v_cache.numel() == 0
    assert nano_qwen_amd.Attention is Attention


def test_no_cpu_fallback():
    key = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        store_kvcache(key, key, cache, cache, torch.tensor([0, 1], dtype=torch.int32))
    q = torch.zeros(2, 1, 32, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        kernels.paged_decode(q, cache, cache, torch.tensor([1, 1], dtype=torch.int32),
                             torch.zeros(2, 1, dtype=torch.int32), 0.1)


def test_store_kvcache_keeps_reference_asserts():
    key = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        store_kvcache(key.transpose(1, 2).contiguous().transpose(1, 2), key, cache, cache,
                      torch.tensor([0, 1], dtype=torch.int32))
    with pytest.raises(AssertionError):
        store_kvcache(key, key, cache, cache, torch.tensor([0], dtype=torch.int32))


def test_runner_prepare_prefill_on_cpu_matches_oracle():
    runner = ModelRunner(block_size=256, max_num_seqs=8, device="cpu")
    rng = np.random.default_rng(3)
    seqs = []
    for i in range(4):
        n = int(rng.integers(1, 1200))
        cached = 256 * int(rng.integers(0, (n - 1) // 256 + 1)) if i % 2 else 0
        sched = n - cached if i != 1 else max(1, (n - cached) // 2)
        seqs.append(Sequence(list(rng.integers(0, 999, n)), block_table=list(rng.permutation(64)[:(n + 255) // 256]),
                             num_cached_tokens=cached, num_scheduled_tokens=sched))
    input_ids, positions = runner.prepare_prefill(seqs)
    md = metadata.prepare_prefill(seqs, 256)
    ctx = C.get_context()
    assert input_ids.tolist() == md["input_ids"] and positions.tolist() == md["positions"]
    assert ctx.slot_mapping.tolist() == md["slot_mapping"]
    assert ctx.cu_seqlens_q.tolist() == md["cu_seqlens_q"] and ctx.cu_seqlens_k.tolist() == md["cu_seqlens_k"]
    assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (md["max_seqlen_q"], md["max_seqlen_k"])
    want = md["block_tables"]
    assert (ctx.block_tables is None) == (want is None)
    if want is not None:
        assert ctx.block_tables.tolist() == want
    assert ctx.slot_mapping.dtype == torch.int32 and ctx.cu_seqlens_q.dtype == torch.int32
    C.reset_context()


def test_runner_allocate_kv_cache_binds_layers():
    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.a = Attention(4, 128, 0.1, 2)
            self.b = Attention(4, 128, 0.1, 2)
    m = M()
    r = ModelRunner(block_size=256, max_num_seqs=4, device="cpu")
    assert r.allocate_kv_cache(m, 2, 3, 2, 128, torch.bfloat16, kv_cache_dtype=torch.float8_e4m3fn) == 2
    assert r.kv_cache.shape == (2, 2, 3, 256, 2, 128)
    assert m.b.k_cache.data_ptr() == r.kv_cache[0, 1].data_ptr()
    assert m.a.k_scale.shape == (2,) and m.b.v_scale.data_ptr() == r.kv_scales[1, 1].data_ptr()


def test_run_model_eager_paths():
    """Prefill and batches above 512 never replay a graph
    (engine/model_runner.py:320); the model's ``compute_logits`` is applied
    when it has one."""
    import torch
    from nano_qwen_amd.engine import ModelRunner
    runner = ModelRunner(block_size=256, max_num_seqs=8, device="cpu")
    runner.graphs = {8: None}    # a replay would fail on this
    runner.graph_bs = [8]
    called = []
    runner.model = lambda i, p: called.append(i.numel()) or torch.zeros(i.numel(), 4)
    ids = torch.zeros(513, dtype=torch.int64)
    assert runner.run_model(ids, ids, False).shape == (513, 4)
    assert runner.run_model(ids[:3], ids[:3], True).shape == (3, 4)
    assert called == [513, 3]

    class WithLogits:
        def __call__(self, i, p):
            return torch.ones(i.numel(), 2)

        def compute_logits(self, h):
            return h * 3
    runner.model = WithLogits()
    runner.enforce_eager = True
    assert torch.equal(runner.run_model(ids[:2], ids[:2], False), torch.full((2, 2), 3.0))


def test_calibrate_kv_scales():
    """absmax/448 per (layer, kv head), in place behind the layers' views;
    all-zero heads keep 1; lists of tensors combine; non-fp8 pools refuse."""
    import pytest
    import torch
    from torch import nn
    from nano_qwen_amd.engine import ModelRunner
    from nano_qwen_amd.layers import Attention
    from oracle.inputs import fp8_scales

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.ModuleList([Attention(4, 16, 0.25, 2) for _ in range(3)])

    model = M()
    runner = ModelRunner(block_size=16, max_num_seqs=4, device="cpu")
    runner.allocate_kv_cache(model, 3, 4, 2, 16, torch.bfloat16, kv_cache_dtype=torch.float8_e4m3fn)
    g = torch.Generator().manual_seed(0)
    kv = []
    for layer in range(3):
        k = torch.randn(37, 2, 16, generator=g).to(torch.bfloat16) * (layer + 1)
        v1 = torch.randn(5, 2, 16, generator=g).to(torch.bfloat16)
        v2 = torch.randn(2, 3, 2, 16, generator=g).to(torch.bfloat16) * 4
        if layer == 2:
            k[:, 1] = 0    # an all-zero head
        kv.append((k, [v1, v2]))
    runner.calibrate_kv_scales(kv)
    for layer, (k, vs) in enumerate(kv):
        assert torch.equal(runner.kv_scales[0, layer], fp8_scales(k))
        assert torch.equal(runner.kv_scales[1, layer], fp8_scales(*vs))
        assert model.a[layer].k_scale.data_ptr() == runner.kv_scales[0, layer].data_ptr()
    assert runner.kv_scales[0, 2, 1].item() == 1.0
    k0 = kv[0][0].float()
    assert torch.allclose(runner.kv_scales[0, 0] * 448, k0.abs().amax(dim=(0, 2)))
    with pytest.raises(ValueError):
        runner.calibrate_kv_scales(kv[:2])
    bf = ModelRunner(block_size=16, max_num_seqs=4, device="cpu")
    bf.allocate_kv_cache(M(), 3, 4, 2, 16, torch.bfloat16)
    with pytest.raises(RuntimeError):
        bf.calibrate_kv_scales(kv)


def test_kv_pool_sized_from_memory_budget():
    """engine/model_runner.py:186-197: blocks = (total * utilization - used -
    peak + current) // block_bytes, block_bytes = 2 L block_size Hkv D
    itemsize -- with the cache dtype's item size, so fp8 gets twice the
    blocks.  Device queries are stood in for; the arithmetic is the
    reference's, restated here in plain integers."""
    from types import SimpleNamespace

    class M(torch.nn.Module):
        def __init__(self, n=3):
            super().__init__()
            self.a = torch.nn.ModuleList([Attention(8, 16, 0.25, 2) for _ in range(n)])

    GiB = 1 << 30
    mem = (30 * GiB, 80 * GiB)                       # free, total
    stats = {"allocated_bytes.all.peak": 7 * GiB, "allocated_bytes.all.current": 5 * GiB}
    L, hkv, d, bs = 3, 2, 16, 16
    r = ModelRunner(block_size=bs, max_num_seqs=4, device="cpu")
    bf_bytes = r.kv_block_bytes(L, hkv, d, torch.bfloat16)
    assert bf_bytes == 2 * L * bs * hkv * d * 2
    budget = int(80 * GiB * 0.5 - (80 - 30) * GiB - 7 * GiB + 5 * GiB)
    assert budget < 0  # 50% of 80 GiB is already used
    assert r.budget_blocks(bf_bytes, 0.5, mem, stats) == budget // bf_bytes
    want_bf = int(80 * GiB * 0.9 - 50 * GiB - 2 * GiB) // bf_bytes
    assert r.budget_blocks(bf_bytes, 0.9, mem, stats) == want_bf
    fp8_bytes = r.kv_block_bytes(L, hkv, d, torch.float8_e4m3fn)
    assert fp8_bytes * 2 == bf_bytes
    assert r.budget_blocks(fp8_bytes, 0.9, mem, stats) in (2 * want_bf, 2 * want_bf + 1)

    # allocate_kv_cache() as the reference calls it: everything from the
    # config and the runner's model, the block count from the budget (a small
    # budget here: the allocation is real host memory)
    small = (50 * GiB + 2 * GiB + 10.5 * bf_bytes) / (80 * GiB)
    hf = SimpleNamespace(num_hidden_layers=L, num_key_value_heads=hkv, head_dim=d, hidden_size=128,
                         num_attention_heads=8, dtype=torch.bfloat16)
    for kv_dtype, blocks in ((None, (10,)), (torch.float8_e4m3fn, (20, 21))):
        cfg = SimpleNamespace(hf_config=hf, gpu_memory_utilization=small, kvcache_block_size=bs, max_num_seqs=4,
                              num_kvcache_blocks=-1, tensor_parallel_size=1, kv_cache_dtype=kv_dtype)
        runner = ModelRunner(device="cpu", config=cfg)
        runner.model = M()
        real_mem, real_stats = torch.cuda.mem_get_info, torch.cuda.memory_stats
        torch.cuda.mem_get_info = lambda device=None: mem
        torch.cuda.memory_stats = lambda device=None: stats
        try:
            assert runner.allocate_kv_cache() == L
        finally:
            torch.cuda.mem_get_info, torch.cuda.memory_stats = real_mem, real_stats
        assert cfg.num_kvcache_blocks in blocks
        assert runner.kv_cache.shape == (2, L, cfg.num_kvcache_blocks, bs, hkv, d)
        assert runner.kv_cache.dtype == (kv_dtype or torch.bfloat16)
    # tensor parallel: each rank holds num_key_value_heads // tp heads
    cfg = SimpleNamespace(hf_config=SimpleNamespace(num_hidden_layers=1, num_key_value_heads=4, hidden_size=64,
                                                    num_attention_heads=4, dtype=torch.bfloat16),
                          gpu_memory_utilization=0.9, kvcache_block_size=16, max_num_seqs=2, num_kvcache_blocks=-1,
                          tensor_parallel_size=2)
    runner = ModelRunner(device="cpu", config=cfg)
    assert runner.allocate_kv_cache(M(1), num_blocks=3) == 1
    assert runner.kv_cache.shape == (2, 1, 3, 16, 2, 16) and cfg.num_kvcache_blocks == 3


def test_release_workspaces_drops_per_stream_buffers():
    kernels._workspaces[(7, 1)] = torch.empty(4)
    kernels._workspaces[(7, 2)] = torch.empty(4)
    kernels._prefill_queues[(7, 1)] = torch.empty(4)
    kernels._retired.append(torch.empty(4))
    try:
        assert kernels.release_workspaces() >= 4
        assert not any(k[0] == 7 for k in kernels._workspaces) and not kernels._retired
    finally:
        for t in (kernels._workspaces, kernels._prefill_queues):
            for k in [k for k in t if k[0] == 7]:
                del t[k]
