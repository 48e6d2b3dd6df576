"""Generate the golden fixtures of this directory.

    python tests/golden/make_golden.py

The reference ships no golden vectors for its paged attention path (its
attention arithmetic lives in the un-vendored flash_attn package), so these
fixtures are small seeded cases whose expected outputs come from the float64
CPU oracle (oracle/), itself pinned in tests/test_oracle.py against torch's
float8 cast, torch SDPA, brute force and closed forms.  They freeze the
oracle's answers (tests/test_golden.py re-derives them on the CPU) and give
the GPU tests fixed inputs with stored expectations (tests/test_gpu_golden.py).

Each file is an .npz (no pickles): 16-bit inputs are stored as their raw
uint16 bit patterns, fp8 as raw bytes, attention expectations as float32
(rounded from the float64 oracle).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import fp8, paged  # noqa: E402


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def values(t):
    return t.to(torch.float64).numpy()


def make_pool(gen, nb, bs, hkv, d, dtype):
    return torch.randn(nb, bs, hkv, d, generator=gen).to(dtype)


def decode_case(seed=11):
    """3 sequences, contexts 1 / 45 / 97 over 32-token blocks (crossing block
    boundaries), GQA 4 -> 2, bf16, scale 1/sqrt(128)."""
    g = torch.Generator().manual_seed(seed)
    bs, hq, hkv, d = 32, 4, 2, 128
    ctx = [1, 45, 97]
    nblk = [(c + bs - 1) // bs for c in ctx]
    pool = sum(nblk) + 2
    perm = torch.randperm(pool, generator=g)
    bt = torch.full((3, max(nblk) + 1), -1, dtype=torch.int32)  # one padding column
    off = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kc = make_pool(g, pool, bs, hkv, d, torch.bfloat16)
    vc = make_pool(g, pool, bs, hkv, d, torch.bfloat16)
    q = torch.randn(3, hq, d, generator=g).to(torch.bfloat16)
    scale = 1.0 / np.sqrt(d)
    out = paged.paged_decode(values(q), values(kc), values(vc), bt.numpy(), np.array(ctx, np.int64), scale)
    np.savez_compressed(os.path.join(HERE, "decode_bf16_small.npz"), q=bits16(q), k_cache=bits16(kc),
                        v_cache=bits16(vc), block_tables=bt.numpy(), context_lens=np.array(ctx, np.int32),
                        scale=np.float64(scale), out=out.astype(np.float32))


def prefill_case(seed=12):
    """3 sequences over a paged cache: (Lq, prefix) = (40, 32), (1, 0),
    (50, 64); GQA 4 -> 2, bf16.  Keys j <= i + P are visible to row i."""
    g = torch.Generator().manual_seed(seed)
    bs, hq, hkv, d = 32, 4, 2, 128
    lq, pre = [40, 1, 50], [32, 0, 64]
    lk = [a + b for a, b in zip(lq, pre)]
    nblk = [(x + bs - 1) // bs for x in lk]
    pool = sum(nblk) + 1
    perm = torch.randperm(pool, generator=g)
    bt = torch.full((3, max(nblk)), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kc = make_pool(g, pool, bs, hkv, d, torch.bfloat16)
    vc = make_pool(g, pool, bs, hkv, d, torch.bfloat16)
    q = torch.randn(sum(lq), hq, d, generator=g).to(torch.bfloat16)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    scale = 1.0 / np.sqrt(d)
    out = paged.varlen_prefill(values(q), values(kc), values(vc), cu_q, cu_k, scale, block_tables=bt.numpy())
    np.savez_compressed(os.path.join(HERE, "prefill_bf16_paged_small.npz"), q=bits16(q), k_cache=bits16(kc),
                        v_cache=bits16(vc), block_tables=bt.numpy(), cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                        scale=np.float64(scale), out=out.astype(np.float32))


def store_fp8_case(seed=13):
    """bf16 K/V rows of 5 tokens (one skipped with slot -1) quantized into an
    e4m3 cache with per-head scales; values span the saturation limit."""
    g = torch.Generator().manual_seed(seed)
    n, hkv, d, bs, nb = 5, 2, 128, 32, 2
    key = (torch.randn(n, hkv, d, generator=g) * 300).to(torch.bfloat16)
    value = (torch.randn(n, hkv, d, generator=g) * 3).to(torch.bfloat16)
    slots = np.array([7, -1, 32, 63, 0], np.int32)
    k_scale = np.array([0.5, 0.75], np.float32)   # key 300 * N(0,1) / 0.5 saturates at 448
    v_scale = np.array([0.01, 0.02], np.float32)
    kq = fp8.quantize(values(key).astype(np.float32), k_scale)
    vq = fp8.quantize(values(value).astype(np.float32), v_scale)
    k_cache = np.zeros((nb, bs, hkv, d), np.uint8)
    v_cache = np.zeros((nb, bs, hkv, d), np.uint8)
    paged.store_kvcache(kq, vq, k_cache, v_cache, slots)
    np.savez_compressed(os.path.join(HERE, "store_fp8_small.npz"), key=bits16(key), value=bits16(value),
                        slot_mapping=slots, k_scale=k_scale, v_scale=v_scale, k_cache=k_cache, v_cache=v_cache)


if __name__ == "__main__":
    decode_case()
    prefill_case()
    store_fp8_case()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
