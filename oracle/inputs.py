"""Seeded synthetic inputs for the five benchmark configurations.

Test infrastructure only.  Every case follows the reference's data layout:
KV pool ``[num_blocks, block_size, Hkv, D]`` (engine/model_runner.py:198),
block tables padded with -1 (:236-240), decode ``slot_mapping`` pointing at
each sequence's next slot and ``context_lens`` counting the new token
(engine/decode_init.py:29-36), prefill ``cu_seqlens_q/k`` with a prefix-cache
hit making ``Lk = P + Lq`` (engine/model_runner.py:251-276).

Integer metadata (lengths, block permutation) is always drawn on the CPU from
``torch.Generator().manual_seed(seed)`` so it is identical whatever device the
values are generated on; float values are drawn on ``device`` from a generator
seeded with ``seed + 1``.
"""
from __future__ import annotations

import math

import torch

# name -> parameters.  "ctx" / "lq" are inclusive uniform ranges.
CONFIGS = {
    "cfg1": dict(kind="decode", hq=16, hkv=8, d=128, bs=256, batch=4, ctx=(128, 512),
                 pool=16, dtype=torch.float32, kv="same", amp=1.0),
    "cfg2": dict(kind="decode", hq=32, hkv=8, d=128, bs=256, batch=64, ctx=(1024, 4096),
                 slack=1.1, dtype=torch.bfloat16, kv="same", amp=0.5),
    "cfg3": dict(kind="prefill", hq=32, hkv=8, d=128, bs=256, nseq=16, lq=(256, 2048),
                 prefix_blocks=(1, 4), slack=1.1, dtype=torch.bfloat16, kv="same", amp=1.0),
    "cfg4": dict(kind="decode", hq=64, hkv=8, d=128, bs=256, batch=8, ctx=(32768, 32768),
                 slack=1.1, min_pool=1024, dtype=torch.bfloat16, kv="same", amp=1.0),
    "cfg5": dict(kind="decode", hq=32, hkv=8, d=128, bs=256, batch=128, ctx=(2048, 8192),
                 slack=1.1, dtype=torch.bfloat16, kv="fp8", amp=1.0),
}

E4M3_MAX = 448.0


def _pool_size(total_blocks, p):
    n = total_blocks
    if "slack" in p:
        n = math.ceil(p["slack"] * total_blocks)
    n = max(n, p.get("min_pool", 0), p.get("pool", 0))
    return n


def _tables(counts, pool, gen):
    """Disjoint block lists from one random permutation of the pool."""
    perm = torch.randperm(pool, generator=gen)
    width = max(counts)
    tables = torch.full((len(counts), width), -1, dtype=torch.int32)
    off = 0
    for i, c in enumerate(counts):
        tables[i, :c] = perm[off:off + c].to(torch.int32)
        off += c
    assert off <= pool
    return tables


def _randn(shape, gen, device, amp, dtype):
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if amp != 1.0:
        x.mul_(amp)
    return x.to(dtype)


def fp8_scales(*tensors):
    """Per-kv-head scale absmax/448 over tensors shaped [..., Hkv, D]."""
    amax = None
    for t in tensors:
        hk = t.shape[-2]
        a = t.float().abs().reshape(-1, hk, t.shape[-1]).amax(dim=(0, 2))
        amax = a if amax is None else torch.maximum(amax, a)
    s = amax / E4M3_MAX
    return torch.where(s > 0, s, torch.ones_like(s)).to(torch.float32)


def quantize_fp8_torch(x, scale):
    """Pool quantization used only to *generate* fp8 inputs (same arithmetic
    as the store kernel: x * (1/scale), saturate, RNE cast)."""
    inv = (1.0 / scale.to(torch.float32)).to(torch.float32)
    y = x.float() * inv.view(*([1] * (x.dim() - 2)), -1, 1)
    return y.clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def make_decode_case(name="cfg2", seed=0, device="cpu", **override):
    """One decode step: new token K/V (stored first) + paged decode over ctx.

    Returns a dict of tensors on ``device``: ``q [B,Hq,D]``, ``k_new/v_new
    [B,Hkv,D]``, ``k_cache/v_cache [NB,BS,Hkv,D]`` (fp8 codes for the fp8
    config, with ``k_scale/v_scale [Hkv]``), ``block_tables [B,W] int32``,
    ``context_lens [B] int32``, ``slot_mapping [B] int32`` and ints.
    """
    p = dict(CONFIGS[name])
    p.update(override)
    cpu = torch.Generator().manual_seed(seed)
    dev = torch.Generator(device=device).manual_seed(seed + 1)
    B, hq, hkv, d, bs = p["batch"], p["hq"], p["hkv"], p["d"], p["bs"]
    lo, hi = p["ctx"]
    ctx = torch.randint(lo, hi + 1, (B,), generator=cpu, dtype=torch.int64)
    counts = [(int(c) + bs - 1) // bs for c in ctx]
    pool = _pool_size(sum(counts), p)
    tables = _tables(counts, pool, cpu)
    slot = torch.tensor([int(tables[b, (int(ctx[b]) - 1) // bs]) * bs + (int(ctx[b]) - 1) % bs
                         for b in range(B)], dtype=torch.int32)
    act = p["dtype"]
    amp = p["amp"]
    k_cache = _randn((pool, bs, hkv, d), dev, device, amp, act)
    v_cache = _randn((pool, bs, hkv, d), dev, device, amp, act)
    q = _randn((B, hq, d), dev, device, amp, act)
    k_new = _randn((B, hkv, d), dev, device, amp, act)
    v_new = _randn((B, hkv, d), dev, device, amp, act)
    case = dict(name=name, kind="decode", hq=hq, hkv=hkv, d=d, block_size=bs, batch=B,
                scale=d ** -0.5, q=q, k_new=k_new, v_new=v_new,
                block_tables=tables.to(device), context_lens=ctx.to(torch.int32).to(device),
                slot_mapping=slot.to(device), num_blocks=pool)
    if p["kv"] == "fp8":
        ks = fp8_scales(k_cache, k_new)
        vs = fp8_scales(v_cache, v_new)
        case["k_cache"] = quantize_fp8_torch(k_cache, ks)
        case["v_cache"] = quantize_fp8_torch(v_cache, vs)
        del k_cache, v_cache
        case["k_scale"], case["v_scale"] = ks, vs
    else:
        case["k_cache"], case["v_cache"] = k_cache, v_cache
        case["k_scale"] = case["v_scale"] = None
    return case


def make_prefill_case(name="cfg3", seed=0, device="cpu", **override):
    """One prefill step: new tokens stored first, then causal varlen attention.

    Even-indexed sequences carry a prefix-cache hit of ``256 * U{1..4}``
    tokens already in the pool, so ``Lk = P + Lq``; when any prefix exists the
    whole batch reads K/V through ``block_tables`` (engine/model_runner.py:275).
    ``override(prefix_blocks=(0, 0))`` makes a batch with no prefix, which
    attention reads from the packed new K/V instead.
    """
    p = dict(CONFIGS[name])
    p.update(override)
    cpu = torch.Generator().manual_seed(seed)
    dev = torch.Generator(device=device).manual_seed(seed + 1)
    n, hq, hkv, d, bs = p["nseq"], p["hq"], p["hkv"], p["d"], p["bs"]
    lo, hi = p["lq"]
    lq = torch.randint(lo, hi + 1, (n,), generator=cpu, dtype=torch.int64).tolist()
    plo, phi = p["prefix_blocks"]
    pre = torch.randint(plo, phi + 1, (n,), generator=cpu, dtype=torch.int64).tolist()
    prefix = [bs * int(pre[i]) if i % 2 == 0 else 0 for i in range(n)]
    lk = [prefix[i] + lq[i] for i in range(n)]
    counts = [(x + bs - 1) // bs for x in lk]
    pool = _pool_size(sum(counts), p)
    tables = _tables(counts, pool, cpu)
    slots = []
    for i in range(n):
        for pos in range(prefix[i], lk[i]):
            slots.append(int(tables[i, pos // bs]) * bs + pos % bs)
    cu_q = [0]
    cu_k = [0]
    for i in range(n):
        cu_q.append(cu_q[-1] + lq[i])
        cu_k.append(cu_k[-1] + lk[i])
    act, amp = p["dtype"], p["amp"]
    total_q = cu_q[-1]
    k_cache = _randn((pool, bs, hkv, d), dev, device, amp, act)
    v_cache = _randn((pool, bs, hkv, d), dev, device, amp, act)
    q = _randn((total_q, hq, d), dev, device, amp, act)
    k_new = _randn((total_q, hkv, d), dev, device, amp, act)
    v_new = _randn((total_q, hkv, d), dev, device, amp, act)
    paged = cu_k[-1] > cu_q[-1]
    case = dict(name=name, kind="prefill", hq=hq, hkv=hkv, d=d, block_size=bs, nseq=n,
                scale=d ** -0.5, q=q, k_new=k_new, v_new=v_new,
                cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=device),
                cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=device),
                max_seqlen_q=max(lq), max_seqlen_k=max(lk), lq=lq, lk=lk, prefix=prefix,
                block_tables=tables.to(device) if paged else None,
                slot_mapping=torch.tensor(slots, dtype=torch.int32, device=device),
                num_blocks=pool)
    if p["kv"] == "fp8":
        ks = fp8_scales(k_cache, k_new)
        vs = fp8_scales(v_cache, v_new)
        case["k_cache"] = quantize_fp8_torch(k_cache, ks)
        case["v_cache"] = quantize_fp8_torch(v_cache, vs)
        case["k_scale"], case["v_scale"] = ks, vs
    else:
        case["k_cache"], case["v_cache"] = k_cache, v_cache
        case["k_scale"] = case["v_scale"] = None
    return case


def decode_bytes(case):
    """Algorithmic HBM bytes of one decode step (store + attention).

    K/V read once per (token, kv head): sum(ctx) * Hkv * D * kv_itemsize * 2;
    Q read and O written once: 2 * B * Hq * D * itemsize; the store reads the
    new K/V and writes them: 2 * 2 * B * Hkv * D (in + cache itemsize);
    metadata: block-table entries used, context_lens, slot_mapping, scales.
    """
    B, hq, hkv, d, bs = case["batch"], case["hq"], case["hkv"], case["d"], case["block_size"]
    ctx = case["context_lens"].to("cpu").to(torch.int64)
    kv_item = case["k_cache"].element_size()
    act_item = case["q"].element_size()
    kv = int(ctx.sum()) * hkv * d * kv_item * 2
    qo = 2 * B * hq * d * act_item
    store = 2 * B * hkv * d * (act_item + kv_item)
    meta = int(((ctx + bs - 1) // bs).sum()) * 4 + B * 4 * 2
    if case.get("k_scale") is not None:
        meta += 2 * hkv * 4
    return kv + qo + store + meta


def decode_flops(case):
    """4 * Hq * D * sum(ctx): QK^T and PV multiply-adds."""
    ctx = case["context_lens"].to("cpu").to(torch.int64)
    return 4 * case["hq"] * case["d"] * int(ctx.sum())


def prefill_flops(case):
    """4 * Hq * D * sum_s [Lq*P + Lq(Lq+1)/2]: unmasked (query, key) pairs."""
    tot = 0
    for lq, lk in zip(case["lq"], case["lk"]):
        p = lk - lq
        tot += lq * p + lq * (lq + 1) // 2
    return 4 * case["hq"] * case["d"] * tot


def prefill_bytes(case):
    """Q read + O written + K/V read once per (key, kv head) + the store."""
    hq, hkv, d = case["hq"], case["hkv"], case["d"]
    tq = sum(case["lq"])
    tk = sum(case["lk"])
    act = case["q"].element_size()
    kv_item = case["k_cache"].element_size()
    return 2 * tq * hq * d * act + 2 * tk * hkv * d * kv_item + 2 * tq * hkv * d * (act + kv_item)


def make_norm_rope_case(name="cfg3", seed=0, device="cpu", rotary_dim=32, max_position=32768):
    """Inputs of the fused q/k norm + rotary + KV store step for the new tokens
    of a prefill (cfg3) or decode (cfg2/cfg4/cfg5) configuration.

    The token set, positions (prefix + 0..Lq-1 per prefill sequence; ctx - 1
    per decode sequence), slots and caches are those of the configuration;
    ``q_gate [N, Hq, 2D]`` stands for ``q_proj``'s output (query | gate per
    head, models/qwen3_5.py:125-126).  Norm weights are U(-1, 1) (Gemma
    weights are centred on 0, layers/layernorm.py docstring) and the table is
    the rope cache of ``rotary_dim`` dims, base 1e7.
    """
    from .qk_norm_rope import rope_cache
    kind = CONFIGS[name]["kind"]
    base = (make_prefill_case if kind == "prefill" else make_decode_case)(name, seed=seed, device=device)
    if kind == "prefill":
        pos = [p + i for p, lq in zip(base["prefix"], base["lq"]) for i in range(lq)]
    else:
        pos = (base["context_lens"].to("cpu").to(torch.int64) - 1).tolist()
    n, hq, hkv, d = len(pos), base["hq"], base["hkv"], base["d"]
    act, amp = CONFIGS[name]["dtype"], CONFIGS[name]["amp"]
    g = torch.Generator(device=device).manual_seed(seed + 2)
    cpu = torch.Generator().manual_seed(seed + 3)
    return dict(name=name, hq=hq, hkv=hkv, d=d, rotary_dim=rotary_dim, n=n,
                q_gate=_randn((n, hq, 2 * d), g, device, amp, act),
                key=base["k_new"], value=base["v_new"],
                q_weight=(torch.rand(d, generator=cpu) * 2 - 1).to(act).to(device),
                k_weight=(torch.rand(d, generator=cpu) * 2 - 1).to(act).to(device),
                positions=torch.tensor(pos, dtype=torch.int64, device=device),
                cos_sin_cache=torch.from_numpy(rope_cache(rotary_dim, max_position, 1e7)).to(device),
                k_cache=base["k_cache"], v_cache=base["v_cache"], slot_mapping=base["slot_mapping"],
                k_scale=base["k_scale"], v_scale=base["v_scale"], eps=1e-6)


def norm_rope_bytes(case):
    """Algorithmic HBM bytes of one fused norm + rotary + store call: q, k, v
    read once; q_out, k_out and the two cache rows written once; each token's
    position, slot and table row; both weights."""
    n, hq, hkv, d, r = case["n"], case["hq"], case["hkv"], case["d"], case["rotary_dim"]
    es = case["key"].element_size()
    ces = case["k_cache"].element_size()
    per_tok = (hq * d + 2 * hkv * d) * es + (hq * d + hkv * d) * es + 2 * hkv * d * ces + 8 + 4 + 4 * r
    return n * per_tok + 2 * d * es
