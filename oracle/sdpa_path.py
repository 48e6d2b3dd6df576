"""CPU baseline of the paged attention path in torch (test/bench only).

The reference's own path cannot run here or on the GPU box (flash_attn is a
CUDA-only third-party library), so the CPU baseline restates it with torch
CPU ops: gather the paged K/V blocks through ``block_tables``
(``index_select``), ``repeat_interleave`` the kv heads by ``G = Hq/Hkv`` and
call ``scaled_dot_product_attention``.  Prefill passes an explicit
bottom-right causal mask, because ``is_causal=True`` is top-left aligned
when ``Lk > Lq``.  fp8 caches are dequantized inside the timed region.

Follows layers/attention.py:59-75 (store, then prefill or decode) and the
semantics stated in ``oracle/paged.py``.  The functions run on whatever
device their tensors are on: the GPU parity tests also use them, in float32
on the device, as the checker of every output row of the full-size configs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def store_kvcache(key, value, k_cache, v_cache, slot_mapping, k_scale=None, v_scale=None):
    """layers/attention.py:33-40 as an ``index_copy_`` over flat rows."""
    n = key.shape[0]
    ok = slot_mapping >= 0
    idx = slot_mapping[ok].to(torch.int64)
    kc = k_cache.view(-1, key.shape[1] * key.shape[2])
    vc = v_cache.view(-1, value.shape[1] * value.shape[2])
    kr = key.reshape(n, -1)[ok]
    vr = value.reshape(n, -1)[ok]
    if k_cache.dtype == torch.float8_e4m3fn:
        hk = key.shape[1]
        kr = (kr.float().view(-1, hk, key.shape[2]) * (1.0 / k_scale).view(1, hk, 1)).clamp(-448, 448)
        vr = (vr.float().view(-1, hk, key.shape[2]) * (1.0 / v_scale).view(1, hk, 1)).clamp(-448, 448)
        # byte views: torch has no fp8 index_copy_ on the device
        kr = kr.reshape(kr.shape[0], -1).to(torch.float8_e4m3fn).view(torch.uint8)
        vr = vr.reshape(vr.shape[0], -1).to(torch.float8_e4m3fn).view(torch.uint8)
        kc, vc = kc.view(torch.uint8), vc.view(torch.uint8)
    kc.index_copy_(0, idx, kr)
    vc.index_copy_(0, idx, vr)


def _gather(cache, table_row, n_keys, scale=None):
    bs = cache.shape[1]
    nblk = (n_keys + bs - 1) // bs
    blk = table_row[:nblk].to(torch.int64)
    x = cache.index_select(0, blk).reshape(-1, cache.shape[2], cache.shape[3])[:n_keys]
    if x.dtype == torch.float8_e4m3fn:
        x = x.float() * scale.view(1, -1, 1)
    return x


def paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale,
                 k_scale=None, v_scale=None, compute_dtype=torch.float32):
    """q [B,Hq,D] -> [B,Hq,D]: per-sequence gather + SDPA (layers/attention.py:71-74)."""
    B, hq, d = q.shape
    hkv = k_cache.shape[2]
    g = hq // hkv
    out = torch.zeros(B, hq, d, dtype=compute_dtype, device=q.device)
    ctx = context_lens.tolist()
    for b in range(B):
        if ctx[b] <= 0:
            continue
        k = _gather(k_cache, block_tables[b], ctx[b], k_scale).to(compute_dtype)
        v = _gather(v_cache, block_tables[b], ctx[b], v_scale).to(compute_dtype)
        k = k.transpose(0, 1).repeat_interleave(g, dim=0).contiguous()        # [Hq, ctx, D]
        v = v.transpose(0, 1).repeat_interleave(g, dim=0).contiguous()
        qq = q[b].to(compute_dtype).unsqueeze(1)                  # [Hq, 1, D]
        out[b] = F.scaled_dot_product_attention(qq, k, v, scale=scale).squeeze(1)
    return out


def varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_tables=None,
                   compute_dtype=torch.float32, k_scale=None, v_scale=None):
    """Causal varlen prefill with a bottom-right mask (layers/attention.py:64-70)."""
    tq, hq, d = q.shape
    hkv = k.shape[-2]
    g = hq // hkv
    cq = cu_seqlens_q.tolist()
    ck = cu_seqlens_k.tolist()
    out = torch.zeros(tq, hq, d, dtype=compute_dtype, device=q.device)
    for s in range(len(cq) - 1):
        lq, lk = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        if lq <= 0:
            continue
        if block_tables is None:
            ks = k[ck[s]:ck[s + 1]]
            vs = v[ck[s]:ck[s + 1]]
        else:
            ks = _gather(k, block_tables[s], lk, k_scale)
            vs = _gather(v, block_tables[s], lk, v_scale)
        ks = ks.to(compute_dtype).transpose(0, 1).repeat_interleave(g, dim=0).contiguous()
        vs = vs.to(compute_dtype).transpose(0, 1).repeat_interleave(g, dim=0).contiguous()
        qs = q[cq[s]:cq[s + 1]].to(compute_dtype).transpose(0, 1).contiguous()          # [Hq, Lq, D]
        p = lk - lq
        mask = torch.arange(lk, device=q.device)[None, :] <= (torch.arange(lq, device=q.device)[:, None] + p)
        o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, scale=scale)
        out[cq[s]:cq[s + 1]] = o.transpose(0, 1)
    return out
