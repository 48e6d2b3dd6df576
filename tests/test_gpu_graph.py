"""Runner-level decode graph capture and replay (engine/model_runner.py:319-336,
421-456): one graph per batch bucket in a shared pool, static ``graph_vars``,
padding rows with ``slot_mapping = -1`` / ``context_lens = 0``.

Each replay is checked three ways: bit for bit against the same model run
eagerly on the same padded inputs, against the float32 SDPA oracle over
the cache it wrote, and on the cache itself (only the batch's new slots
change; padding rows store nothing and decode to zeros)."""
import numpy as np
import pytest
import torch
from torch import nn

from nano_qwen_amd.engine import ModelRunner, Sequence
from nano_qwen_amd.layers import Attention
from nano_qwen_amd.utils.context import reset_context, set_context
from oracle import sdpa_path
from tests.parity import TOL_BF16, TOL_FP8, assert_close

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 256
L, VOCAB, NB, MAX_BLOCKS = 2, 512, 200, 4


class EmbedAttn(nn.Module):
    """Per layer: q/k/v rows looked up by token id (q scaled by a function of
    the position), attention through the context, outputs summed over the
    layers -> ``[N, Hq * D]``."""

    def __init__(self, device, seed=0):
        super().__init__()
        g = torch.Generator(device=device).manual_seed(seed)
        self.wq = (torch.randn(L, VOCAB, HQ, D, generator=g, device=device) * 0.5).to(torch.bfloat16)
        self.wk = torch.randn(L, VOCAB, HKV, D, generator=g, device=device).to(torch.bfloat16)
        self.wv = torch.randn(L, VOCAB, HKV, D, generator=g, device=device).to(torch.bfloat16)
        self.attn = nn.ModuleList([Attention(HQ, D, D ** -0.5, HKV) for _ in range(L)])

    def qkv(self, layer, input_ids, positions):
        q = self.wq[layer].index_select(0, input_ids)
        q = q * (1.0 + 0.01 * (positions % 11)).to(q.dtype)[:, None, None]
        return q, self.wk[layer].index_select(0, input_ids), self.wv[layer].index_select(0, input_ids)

    def forward(self, input_ids, positions):
        out = None
        for li, layer in enumerate(self.attn):
            o = layer(*self.qkv(li, input_ids, positions)).reshape(input_ids.size(0), HQ * D)
            out = o if out is None else out + o
        return out


def _batch(rng, runner, bs):
    blocks = list(rng.permutation(NB))
    seqs = []
    for _ in range(bs):
        ctx = int(rng.integers(1, BS * MAX_BLOCKS))
        table = [int(blocks.pop()) for _ in range((ctx + BS - 1) // BS)]
        seqs.append(Sequence(list(rng.integers(0, VOCAB, ctx)), block_table=table))
    runner.sampled_token_ids_gpu[:bs] = torch.tensor([s.last_token for s in seqs], device=runner.device)
    return seqs


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_decode_graph_buckets(cuda, kv_dtype):
    rng = np.random.default_rng(3)
    fp8 = kv_dtype == torch.float8_e4m3fn
    model = EmbedAttn(cuda)
    runner = ModelRunner(block_size=BS, max_num_seqs=40, device=cuda)
    assert runner.allocate_kv_cache(model, L, NB, HKV, D, torch.bfloat16, kv_cache_dtype=kv_dtype) == L
    g = torch.Generator(device=cuda).manual_seed(5)
    runner.kv_cache.view(torch.uint8).copy_(
        torch.randint(0, 120, runner.kv_cache.view(torch.uint8).shape, generator=g, dtype=torch.uint8,
                      device=cuda))
    if fp8:
        runner.kv_scales.copy_(torch.rand(2, L, HKV, generator=g, device=cuda) * 0.02 + 0.005)
    else:
        runner.kv_cache.copy_(torch.randn(runner.kv_cache.shape, generator=g, device=cuda).to(kv_dtype))
    before_capture = runner.kv_cache.clone()
    runner.capture_cudagraph(model, HQ * D, max_model_len=BS * MAX_BLOCKS, dtype=torch.bfloat16)
    assert runner.graph_bs == [1, 2, 4, 8, 16, 32, 40]
    assert sorted(runner.graphs) == runner.graph_bs
    # capturing stored nothing (its slot_mapping is all -1)
    assert torch.equal(runner.kv_cache.view(torch.uint8), before_capture.view(torch.uint8))
    tol = TOL_FP8 if fp8 else TOL_BF16
    for bs in (1, 3, 13, 40, 5, 32):
        seqs = _batch(rng, runner, bs)
        input_ids, positions = runner.prepare_decode(seqs)
        ctx = runner.decode_gpu
        slots = ctx["slot_mapping"][:bs].clone()
        pre = runner.kv_cache.clone()
        print(f"graph replay bs={bs} kv={kv_dtype}", flush=True)
        out_g = runner.run_model(input_ids, positions, False).clone()
        torch.cuda.synchronize()
        bucket = next(x for x in runner.graph_bs if x >= bs)
        gv = runner.graph_vars
        assert out_g.shape == (bs, HQ * D)
        # padding rows decode to zeros
        assert (gv["outputs"][bs:bucket] == 0).all()
        post = runner.kv_cache.clone()

        # the cache: the oracle's store of this batch's k/v into `pre`
        expect = pre.clone()
        for li in range(L):
            _, k, v = model.qkv(li, input_ids, positions)
            sdpa_path.store_kvcache(k, v, expect[0, li], expect[1, li], slots,
                                    runner.kv_scales[0, li] if fp8 else None,
                                    runner.kv_scales[1, li] if fp8 else None)
        assert torch.equal(post.view(torch.uint8), expect.view(torch.uint8)), f"cache after bs={bs}"

        # eager on the same padded inputs, from the same cache: bit-identical
        runner.kv_cache.copy_(pre)
        set_context(False, slot_mapping=gv["slot_mapping"][:bucket], context_lens=gv["context_lens"][:bucket],
                    block_tables=gv["block_tables"][:bucket])
        out_e = model(gv["input_ids"][:bucket], gv["positions"][:bucket])
        torch.cuda.synchronize()
        reset_context()
        assert torch.equal(out_g, out_e[:bs]), f"replay != eager at bs={bs}"
        assert torch.equal(runner.kv_cache.view(torch.uint8), post.view(torch.uint8))

        # the oracle over the cache the replay wrote
        ref = torch.zeros(bs, HQ, D, dtype=torch.float32, device=cuda)
        bt = torch.tensor([s.block_table + [0] * (MAX_BLOCKS - len(s.block_table)) for s in seqs],
                          dtype=torch.int32, device=cuda)
        cl = torch.tensor([len(s) for s in seqs], dtype=torch.int32, device=cuda)
        for li in range(L):
            q, _, _ = model.qkv(li, input_ids, positions)
            ref += sdpa_path.paged_decode(q.float(), post[0, li], post[1, li], bt, cl, D ** -0.5,
                                          runner.kv_scales[0, li] if fp8 else None,
                                          runner.kv_scales[1, li] if fp8 else None)
        # the output is the bf16 sum of L layers' outputs: L times the bound of one
        assert_close(out_g.view(bs, HQ, D).float().cpu().numpy(), ref.cpu().numpy(), what=f"graph bs={bs}",
                     max_abs=L * tol["max_abs"], mean_abs=L * tol["mean_abs"])

