"""End to end through the drop-in surface: ModelRunner.prepare_prefill /
prepare_decode -> set_context -> Attention.forward (layers/attention.py:59-75,
engine/model_runner.py:242-306)."""
import numpy as np
import pytest
import torch
from torch import nn

from nano_qwen_amd.engine import ModelRunner, Sequence
from nano_qwen_amd.layers import Attention
from nano_qwen_amd.layers.attention import store_kvcache
from nano_qwen_amd.utils.context import get_context, reset_context
from oracle import metadata, paged
from tests.parity import TOL_BF16, TOL_FP8, assert_close, f64

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 256


class TwoLayers(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = nn.ModuleList([Attention(HQ, D, D ** -0.5, HKV) for _ in range(2)])


def _seqs(rng, n, with_prefix):
    seqs = []
    free = list(rng.permutation(200))
    for i in range(n):
        L = int(rng.integers(1, 900))
        cached = BS * int(rng.integers(1, 3)) if (with_prefix and i % 2 == 0) else 0
        total = cached + L
        table = [int(free.pop()) for _ in range((total + BS - 1) // BS)]
        seqs.append(Sequence(list(rng.integers(0, 1000, total)), block_table=table,
                             num_cached_tokens=cached, num_scheduled_tokens=L))
    return seqs


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_runner_prefill_then_decode(cuda, kv_dtype):
    rng = np.random.default_rng(0)
    model = TwoLayers()
    runner = ModelRunner(block_size=BS, max_num_seqs=16, device=cuda)
    assert runner.allocate_kv_cache(model, 2, 200, HKV, D, torch.bfloat16, kv_cache_dtype=kv_dtype) == 2
    runner.kv_cache.view(torch.uint8).zero_()
    fp8 = kv_dtype == torch.float8_e4m3fn
    if fp8:
        runner.kv_scales.copy_(torch.rand(2, 2, HKV, device=cuda) * 0.02 + 0.005)
    seqs = _seqs(rng, 5, with_prefix=True)
    # pre-existing prefix content of the cache (as if a previous request wrote it)
    runner.kv_cache.view(torch.uint8).copy_(
        torch.randint(0, 120, runner.kv_cache.view(torch.uint8).shape, dtype=torch.uint8, device=cuda))
    if not fp8:
        runner.kv_cache.copy_(torch.randn_like(runner.kv_cache, dtype=torch.float32).to(kv_dtype))
    pre = runner.kv_cache.clone()

    input_ids, positions = runner.prepare_prefill(seqs)
    ctx = get_context()
    md = metadata.prepare_prefill(seqs, BS)
    assert ctx.is_prefill and ctx.block_tables is not None
    assert ctx.cu_seqlens_q.tolist() == md["cu_seqlens_q"] and ctx.cu_seqlens_k.tolist() == md["cu_seqlens_k"]
    assert ctx.slot_mapping.tolist() == md["slot_mapping"] and positions.tolist() == md["positions"]
    assert ctx.block_tables.tolist() == md["block_tables"]
    T = len(md["slot_mapping"])
    g = torch.Generator(device=cuda).manual_seed(1)
    q = torch.randn(T, HQ, D, generator=g, device=cuda).to(torch.bfloat16)
    k = torch.randn(T, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn(T, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    outs = [layer(q, k, v) for layer in model.attn]
    torch.cuda.synchronize()
    tol = TOL_FP8 if fp8 else TOL_BF16
    for li, o in enumerate(outs):
        kc, vc = f64(pre[0, li]), f64(pre[1, li])
        ks = vs = None
        if fp8:
            from oracle import fp8 as F8
            ks, vs = runner.kv_scales[0, li].cpu().numpy(), runner.kv_scales[1, li].cpu().numpy()
            kq, vq = F8.quantize(k.float().cpu().numpy(), ks), F8.quantize(v.float().cpu().numpy(), vs)
            kc_u, vc_u = pre[0, li].view(torch.uint8).cpu().numpy().copy(), pre[1, li].view(torch.uint8).cpu().numpy().copy()
            paged.store_kvcache(kq, vq, kc_u, vc_u, np.array(md["slot_mapping"]))
            kc, vc = F8.decode_e4m3fn(kc_u).astype(np.float64), F8.decode_e4m3fn(vc_u).astype(np.float64)
            assert np.array_equal(runner.kv_cache[0, li].view(torch.uint8).cpu().numpy(), kc_u)
        else:
            paged.store_kvcache(f64(k), f64(v), kc, vc, np.array(md["slot_mapping"]))
        ref = paged.varlen_prefill(f64(q), kc, vc, md["cu_seqlens_q"], md["cu_seqlens_k"], D ** -0.5,
                                   block_tables=np.array(md["block_tables"]), k_scale=ks, v_scale=vs)
        assert_close(f64(o), ref, **tol, what=f"prefill layer {li}")

    # ---- one decode step for every sequence
    for s in seqs:
        s.num_cached_tokens = len(s)
        s.append_token(7)
        if len(s) > len(s.block_table) * BS:
            s.block_table.append(150 + s.seq_id % 40)
    runner.sampled_token_ids_gpu.copy_(torch.arange(16, device=cuda) * 11)
    runner.batch_slots_gpu[:5] = torch.tensor([3, 1, 4, 0, 2], device=cuda)
    pre = runner.kv_cache.clone()
    input_ids, positions = runner.prepare_decode(seqs)
    ctx = get_context()
    mdd = metadata.prepare_decode(seqs, BS, sampled_token_ids=np.arange(16) * 11, batch_slots=[3, 1, 4, 0, 2])
    assert not ctx.is_prefill
    assert ctx.context_lens.tolist() == mdd["context_lens"] and ctx.slot_mapping.tolist() == mdd["slot_mapping"]
    assert positions.tolist() == mdd["positions"] and input_ids.tolist() == mdd["input_ids"]
    qd = torch.randn(5, HQ, D, generator=g, device=cuda).to(torch.bfloat16)
    kd = torch.randn(5, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    vd = torch.randn(5, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    o = model.attn[0](qd, kd, vd)
    torch.cuda.synchronize()
    assert o.shape == (5, 1, HQ, D)
    kc, vc = f64(pre[0, 0]), f64(pre[1, 0])
    ks = vs = None
    if fp8:
        from oracle import fp8 as F8
        ks, vs = runner.kv_scales[0, 0].cpu().numpy(), runner.kv_scales[1, 0].cpu().numpy()
        kc_u, vc_u = pre[0, 0].view(torch.uint8).cpu().numpy().copy(), pre[1, 0].view(torch.uint8).cpu().numpy().copy()
        paged.store_kvcache(F8.quantize(kd.float().cpu().numpy(), ks), F8.quantize(vd.float().cpu().numpy(), vs),
                            kc_u, vc_u, np.array(mdd["slot_mapping"]))
        kc, vc = F8.decode_e4m3fn(kc_u).astype(np.float64), F8.decode_e4m3fn(vc_u).astype(np.float64)
    else:
        paged.store_kvcache(f64(kd), f64(vd), kc, vc, np.array(mdd["slot_mapping"]))
    ref = paged.paged_decode(f64(qd), kc, vc, np.array(mdd["block_tables"]), np.array(mdd["context_lens"]),
                             D ** -0.5, ks, vs)
    assert_close(f64(o[:, 0]), ref, **tol, what="decode")
    reset_context()


def test_runner_warmup_prefill_without_cache(cuda):
    """Warmup runs a prefill before the KV cache exists: no store, packed K/V
    (layers/attention.py:62, engine/model_runner.py:171-184)."""
    attn = Attention(HQ, D, D ** -0.5, HKV)
    runner = ModelRunner(block_size=BS, max_num_seqs=4, device=cuda)
    seqs = [Sequence([0] * 300, num_scheduled_tokens=300), Sequence([0] * 77, num_scheduled_tokens=77)]
    runner.prepare_prefill(seqs)
    ctx = get_context()
    assert ctx.block_tables is None and ctx.slot_mapping.numel() == 0
    g = torch.Generator(device=cuda).manual_seed(0)
    q = torch.randn(377, HQ, D, generator=g, device=cuda).to(torch.bfloat16)
    k = torch.randn(377, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn(377, HKV, D, generator=g, device=cuda).to(torch.bfloat16)
    o = attn(q, k, v)
    torch.cuda.synchronize()
    ref = paged.varlen_prefill(f64(q), f64(k), f64(v), [0, 300, 377], [0, 300, 377], D ** -0.5)
    assert_close(f64(o), ref, **TOL_BF16, what="warmup prefill")
    reset_context()


def test_calibrated_fp8_store_uses_full_range(cuda):
    """After ``calibrate_kv_scales`` on a batch's new K/V, the HIP store of
    that batch puts each (layer, kv head)'s absmax element at e4m3's largest
    finite value, +-448, and nothing beyond: the scale spends the whole range
    without saturating."""
    model = TwoLayers()
    runner = ModelRunner(block_size=BS, max_num_seqs=4, device=cuda)
    runner.allocate_kv_cache(model, 2, 8, HKV, D, torch.bfloat16, kv_cache_dtype=torch.float8_e4m3fn)
    runner.kv_cache.view(torch.uint8).zero_()
    g = torch.Generator(device=cuda).manual_seed(2)
    n = 300
    kv = [(torch.randn(n, HKV, D, generator=g, device=cuda).to(torch.bfloat16) * (li + 1),
           torch.randn(n, HKV, D, generator=g, device=cuda).to(torch.bfloat16) * 0.1) for li in range(2)]
    runner.calibrate_kv_scales(kv)
    slots = torch.arange(n, dtype=torch.int32, device=cuda) + 17
    for li, layer in enumerate(model.attn):
        k, v = kv[li]
        store_kvcache(k, v, layer.k_cache, layer.v_cache, slots, layer.k_scale, layer.v_scale)
    torch.cuda.synchronize()
    for li in range(2):
        for which in range(2):
            codes = runner.kv_cache[which, li].reshape(-1, HKV, D)[17:17 + n].float()
            amax = codes.abs().amax(dim=(0, 2))
            assert torch.all(amax == 448.0), (li, which, amax)
            deq = codes * runner.kv_scales[which, li].view(1, HKV, 1)
            x = kv[li][which].float()
            # e4m3 keeps 3 mantissa bits: relative error at most 2^-4, plus the subnormal step
            assert torch.all((deq - x).abs() <= x.abs() * 2.0 ** -4 + runner.kv_scales[which, li].view(1, HKV, 1) * 2.0 ** -10)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_runner_pool_from_memory_budget(cuda, kv_dtype):
    """allocate_kv_cache() sized from the device's memory budget
    (engine/model_runner.py:186-197): a utilization that leaves room for
    about 1 GiB of bf16 blocks; fp8 gets twice the blocks of the same
    budget, and the pool's last block stores and decodes."""
    from types import SimpleNamespace
    torch.cuda.synchronize()
    free, total = torch.cuda.mem_get_info(cuda)
    st = torch.cuda.memory_stats(cuda)
    reserve = (total - free) + st["allocated_bytes.all.peak"] - st["allocated_bytes.all.current"]
    util = (reserve + (1 << 30)) / total
    hf = SimpleNamespace(num_hidden_layers=2, num_key_value_heads=HKV, head_dim=D, hidden_size=HQ * D,
                         num_attention_heads=HQ, dtype=torch.bfloat16)
    cfg = SimpleNamespace(hf_config=hf, gpu_memory_utilization=util, kvcache_block_size=BS, max_num_seqs=4,
                          num_kvcache_blocks=-1, tensor_parallel_size=1, kv_cache_dtype=kv_dtype)
    runner = ModelRunner(device=cuda, config=cfg)
    runner.model = TwoLayers()
    bf16_bytes = runner.kv_block_bytes(2, HKV, D, torch.bfloat16)
    print(f"[budget] {kv_dtype} util {util:.4f} of {total / 2**30:.1f} GiB", flush=True)
    assert runner.allocate_kv_cache() == 2
    nb = cfg.num_kvcache_blocks
    want = (1 << 30) // bf16_bytes * (2 if kv_dtype == torch.float8_e4m3fn else 1)
    assert abs(nb - want) <= 2 + want // 50, (nb, want)   # other allocations may move in between
    assert runner.kv_cache.shape == (2, 2, nb, BS, HKV, D) and runner.kv_cache.dtype == kv_dtype
    # one decode step whose only block is the pool's last one
    attn = runner.model.attn[0]
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, HKV, D, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(1, HKV, D, generator=g).to(torch.bfloat16).to(cuda)
    q = torch.randn(1, HQ, D, generator=g).to(torch.bfloat16).to(cuda)
    if kv_dtype == torch.float8_e4m3fn:
        runner.kv_scales.fill_(0.02)
    slot = torch.tensor([(nb - 1) * BS], dtype=torch.int32, device=cuda)
    store_kvcache(k, v, attn.k_cache, attn.v_cache, slot, attn.k_scale, attn.v_scale)
    from nano_qwen_amd import kernels
    out = kernels.paged_decode(q.unsqueeze(1), attn.k_cache, attn.v_cache,
                               torch.tensor([1], dtype=torch.int32, device=cuda),
                               torch.tensor([[nb - 1]], dtype=torch.int32, device=cuda), D ** -0.5,
                               attn.k_scale, attn.v_scale)
    torch.cuda.synchronize()
    # one token: every head's output is its kv head's stored V row
    vs = attn.v_cache[nb - 1, 0].float()
    if kv_dtype == torch.float8_e4m3fn:
        vs = vs * attn.v_scale.view(-1, 1)
    ref = vs.repeat_interleave(HQ // HKV, dim=0)
    assert torch.allclose(out[0, 0].float(), ref, atol=1e-2, rtol=1e-2)
    for m in runner.model.attn:
        m.k_cache = m.v_cache = torch.tensor([])
    runner.kv_cache = runner.kv_scales = None
    del attn
    torch.cuda.empty_cache()
