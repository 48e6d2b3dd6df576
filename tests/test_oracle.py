"""Pin the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something independent of its own
formula: a library routine (torch's float8 cast, torch SDPA), a pure-Python
brute force, closed-form special cases, or invariants that a plausible
mistake (wrong GQA index, top-left instead of bottom-right causal alignment,
wrong block-table indexing, dropped scale) would break.
"""
import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8, metadata, paged, sdpa_path
from oracle.inputs import make_decode_case, make_prefill_case

# ----------------------------------------------------------------- fp8 codec


def test_fp8_decode_all_codes_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = fp8.decode_e4m3fn(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert fp8.decode_e4m3fn(np.array([0x7E], np.uint8))[0] == 448.0
    assert fp8.decode_e4m3fn(np.array([0x01], np.uint8))[0] == 2.0 ** -9


def test_fp8_encode_roundtrip_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.decode_e4m3fn(codes)
    fin = ~np.isnan(vals)
    back = fp8.encode_e4m3fn(vals[fin])
    assert np.array_equal(back, codes[fin])


def test_fp8_encode_matches_torch_cast_exhaustive_bf16():
    # every bf16 bit pattern, saturated to +-448 first (torch turns overflow
    # into NaN, the quantizer saturates)
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    y = np.minimum(np.maximum(x, np.float32(-448)), np.float32(448)).astype(np.float32)
    ours = fp8.encode_e4m3fn(y)
    ref = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_fp8_encode_matches_torch_cast_random_f32_and_ties():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * rng.choice([1e-3, 1e-2, 1, 30, 300], 200000)).astype(np.float32)
    # exact midpoints between neighbouring codes: ties must go to the even code
    grid = fp8.decode_e4m3fn(np.arange(0, 127, dtype=np.uint8)).astype(np.float64)
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids]).astype(np.float32)
    y = np.clip(x, -448, 448).astype(np.float32)
    ours = fp8.encode_e4m3fn(y)
    ref = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    # midpoint of codes 1 and 2 (odd, even) rounds to 2; of 2 and 3 rounds to 2
    assert fp8.encode_e4m3fn(np.float32([(2 ** -9 + 2 ** -8) / 2]))[0] == 2
    assert fp8.encode_e4m3fn(np.float32([(2 ** -8 + 3 * 2 ** -9) / 2]))[0] == 2


def test_fp8_quantize_scale_and_saturation():
    x = np.array([[[0.5, -1.0, 1000.0, -1000.0]]], dtype=np.float32)  # [1, 1 head, 4]
    s = np.array([1.0 / 128], dtype=np.float32)
    q = fp8.quantize(x, s)
    v = fp8.decode_e4m3fn(q)
    assert v.tolist() == [[[64.0, -128.0, 448.0, -448.0]]]
    assert fp8.quantize(np.float32([[[np.nan]]]), np.float32([1]))[0, 0, 0] & 0x7F == 0x7F


# ----------------------------------------------------------------- store


def test_store_kvcache_closed_form_and_skip():
    rng = np.random.default_rng(1)
    nb, bs, hkv, d, n = 6, 16, 2, 8, 9
    kc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    k0, v0 = kc.copy(), vc.copy()
    key = rng.standard_normal((n, hkv, d)).astype(np.float32)
    val = rng.standard_normal((n, hkv, d)).astype(np.float32)
    slots = rng.choice(nb * bs, n, replace=False).astype(np.int32)
    slots[[2, 5]] = -1
    paged.store_kvcache(key, val, kc, vc, slots)
    for i in range(n):
        if slots[i] < 0:
            continue
        b, o = divmod(int(slots[i]), bs)
        assert np.array_equal(kc[b, o], key[i]) and np.array_equal(vc[b, o], val[i])
    touched = np.zeros(nb * bs, bool)
    touched[slots[slots >= 0]] = True
    assert np.array_equal(kc.reshape(nb * bs, -1)[~touched], k0.reshape(nb * bs, -1)[~touched])
    assert np.array_equal(vc.reshape(nb * bs, -1)[~touched], v0.reshape(nb * bs, -1)[~touched])


def test_store_kvcache_matches_torch_index_copy():
    case = make_decode_case("cfg1", seed=3)
    kc, vc = case["k_cache"].clone(), case["v_cache"].clone()
    sdpa_path.store_kvcache(case["k_new"], case["v_new"], kc, vc, case["slot_mapping"])
    kn, vn = case["k_cache"].numpy().copy(), case["v_cache"].numpy().copy()
    paged.store_kvcache(case["k_new"].numpy(), case["v_new"].numpy(), kn, vn, case["slot_mapping"].numpy())
    assert np.array_equal(kc.numpy(), kn) and np.array_equal(vc.numpy(), vn)


# ----------------------------------------------------------------- attention


def _brute_decode(q, kc, vc, bt, ctx, scale):
    """Pure-Python loops (tiny shapes only)."""
    B, hq, d = q.shape
    bs, hkv = kc.shape[1], kc.shape[2]
    g = hq // hkv
    out = np.zeros((B, hq, d))
    for b in range(B):
        for h in range(hq):
            kvh = h // g
            scores = []
            for j in range(int(ctx[b])):
                blk, off = int(bt[b][j // bs]), j % bs
                scores.append(sum(float(q[b, h, t]) * float(kc[blk, off, kvh, t]) for t in range(d)) * scale)
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            z = sum(w)
            for j in range(int(ctx[b])):
                blk, off = int(bt[b][j // bs]), j % bs
                for t in range(d):
                    out[b, h, t] += w[j] / z * float(vc[blk, off, kvh, t])
    return out


def _tiny_decode(seed=0, B=3, hq=4, hkv=2, d=4, bs=8, nb=10, ctx=(1, 20)):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, hq, d))
    kc = rng.standard_normal((nb, bs, hkv, d))
    vc = rng.standard_normal((nb, bs, hkv, d))
    lens = rng.integers(ctx[0], ctx[1] + 1, B)
    perm = rng.permutation(nb)
    W = max(-(-int(c) // bs) for c in lens)
    bt = -np.ones((B, W), np.int64)
    off = 0
    for b in range(B):
        c = -(-int(lens[b]) // bs)
        bt[b, :c] = perm[off:off + c]
        off += c
    return q, kc, vc, bt, lens


def test_decode_matches_bruteforce_tiny():
    q, kc, vc, bt, lens = _tiny_decode(B=3, ctx=(5, 19))  # crosses block boundaries
    ours = paged.paged_decode(q, kc, vc, bt, lens, 0.37)
    ref = _brute_decode(q, kc, vc, bt, lens, 0.37)
    np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-12)


def test_decode_matches_torch_sdpa_f64():
    case = make_decode_case("cfg1", seed=0)
    q = case["q"].double()
    kc, vc = case["k_cache"].double(), case["v_cache"].double()
    bt, ctx = case["block_tables"], case["context_lens"]
    ours = paged.paged_decode(q.numpy(), kc.numpy(), vc.numpy(), bt.numpy(), ctx.numpy(), case["scale"])
    ref = sdpa_path.paged_decode(q, kc, vc, bt, ctx, case["scale"], compute_dtype=torch.float64)
    np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-9, atol=1e-11)


def test_decode_gqa_head_mapping():
    # Hq=4, Hkv=2: heads 0,1 -> kv 0 and 2,3 -> kv 1 (h // G), not h % Hkv.
    q, kc, vc, bt, lens = _tiny_decode(B=1, hq=4, hkv=2, ctx=(9, 9))
    vc[..., 0, :] = 1.0
    vc[..., 1, :] = -1.0
    out = paged.paged_decode(q, kc, vc, bt, lens, 0.5)
    np.testing.assert_allclose(out[0, :2], 1.0)
    np.testing.assert_allclose(out[0, 2:], -1.0)


def test_decode_special_cases():
    q, kc, vc, bt, lens = _tiny_decode(B=2, ctx=(1, 1))
    out = paged.paged_decode(q, kc, vc, bt, lens, 0.5)        # ctx=1: o = v[0]
    for b in range(2):
        np.testing.assert_allclose(out[b], np.repeat(vc[bt[b, 0], 0], 2, axis=0))
    q, kc, vc, bt, lens = _tiny_decode(B=2, ctx=(13, 13))
    out = paged.paged_decode(np.zeros_like(q), kc, vc, bt, lens, 0.5)   # q=0: mean of V
    for b in range(2):
        V = paged.gather_keys(vc, bt[b], 13)
        np.testing.assert_allclose(out[b], np.repeat(V.mean(0), 2, axis=0), rtol=1e-12)
    # one dominant key selects its value row
    q, kc, vc, bt, lens = _tiny_decode(B=1, hq=2, hkv=1, d=4, ctx=(11, 11))
    q[:] = 0
    q[0, :, 0] = 1.0
    blk, off = bt[0, 7 // 8], 7 % 8
    kc[blk, off, 0, 0] = 1e4
    out = paged.paged_decode(q, kc, vc, bt, lens, 1.0)
    np.testing.assert_allclose(out[0, 0], vc[blk, off, 0], rtol=1e-12)


def test_decode_block_permutation_invariance():
    q, kc, vc, bt, lens = _tiny_decode(seed=4, B=3, nb=12, ctx=(9, 30))
    out = paged.paged_decode(q, kc, vc, bt, lens, 0.3)
    perm = np.random.default_rng(9).permutation(kc.shape[0])
    inv = np.argsort(perm)
    kc2, vc2 = kc[perm], vc[perm]          # physical block p now holds old block perm[p]
    bt2 = np.where(bt >= 0, inv[np.maximum(bt, 0)], -1)
    out2 = paged.paged_decode(q, kc2, vc2, bt2, lens, 0.3)
    assert np.array_equal(out, out2)


def test_decode_ignores_table_padding_and_zero_ctx():
    q, kc, vc, bt, lens = _tiny_decode(seed=5, B=3, ctx=(3, 17))
    out = paged.paged_decode(q, kc, vc, bt, lens, 0.3)
    bt2 = np.concatenate([bt, np.full((3, 4), 7)], axis=1)   # stale entries past ctx
    out2 = paged.paged_decode(q, kc, vc, bt2, lens, 0.3)
    assert np.array_equal(out, out2)
    lens0 = lens.copy()
    lens0[1] = 0
    out3 = paged.paged_decode(q, kc, vc, bt, lens0, 0.3)
    assert np.all(out3[1] == 0) and np.array_equal(out3[0], out[0])


def test_prefill_p0_matches_sdpa_is_causal():
    rng = np.random.default_rng(6)
    lens = [5, 17, 1]
    cu = np.cumsum([0] + lens)
    hq, hkv, d = 4, 2, 8
    q = rng.standard_normal((cu[-1], hq, d))
    k = rng.standard_normal((cu[-1], hkv, d))
    v = rng.standard_normal((cu[-1], hkv, d))
    ours = paged.varlen_prefill(q, k, v, cu, cu, 0.4)
    for s in range(3):
        qs = torch.from_numpy(q[cu[s]:cu[s + 1]]).transpose(0, 1)
        ks = torch.from_numpy(k[cu[s]:cu[s + 1]]).transpose(0, 1).repeat_interleave(2, 0)
        vs = torch.from_numpy(v[cu[s]:cu[s + 1]]).transpose(0, 1).repeat_interleave(2, 0)
        ref = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True, scale=0.4).transpose(0, 1)
        np.testing.assert_allclose(ours[cu[s]:cu[s + 1]], ref.numpy(), rtol=1e-9, atol=1e-11)


def test_prefill_bottom_right_alignment_bruteforce():
    # Lk > Lq: row i sees keys j <= i + (Lk - Lq); top-left alignment would not.
    rng = np.random.default_rng(7)
    lq, lk, hq, hkv, d = 3, 7, 2, 1, 4
    q = rng.standard_normal((lq, hq, d))
    k = rng.standard_normal((lk, hkv, d))
    v = rng.standard_normal((lk, hkv, d))
    ours = paged.varlen_prefill(q, k, v, [0, lq], [0, lk], 0.5)
    for i in range(lq):
        for h in range(hq):
            n = i + (lk - lq) + 1
            s = [sum(q[i, h, t] * k[j, 0, t] for t in range(d)) * 0.5 for j in range(n)]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            z = sum(w)
            ref = [sum(w[j] / z * v[j, 0, t] for j in range(n)) for t in range(d)]
            np.testing.assert_allclose(ours[i, h], ref, rtol=1e-12)


def test_prefill_paged_equals_packed_and_decode_is_last_row():
    case = make_prefill_case("cfg3", seed=2, nseq=4, lq=(3, 40), prefix_blocks=(1, 2), bs=16,
                             hq=4, hkv=2, d=8, dtype=torch.float64)
    kc, vc = case["k_cache"].numpy().copy(), case["v_cache"].numpy().copy()
    paged.store_kvcache(case["k_new"].numpy(), case["v_new"].numpy(), kc, vc, case["slot_mapping"].numpy())
    bt = case["block_tables"].numpy()
    cq, ck = case["cu_seqlens_q"].numpy(), case["cu_seqlens_k"].numpy()
    out = paged.varlen_prefill(case["q"].numpy(), kc, vc, cq, ck, 0.3, block_tables=bt)
    # packed equivalent: gather each sequence's keys contiguously
    ks = np.concatenate([paged.gather_keys(kc, bt[s], ck[s + 1] - ck[s]) for s in range(4)])
    vs = np.concatenate([paged.gather_keys(vc, bt[s], ck[s + 1] - ck[s]) for s in range(4)])
    out2 = paged.varlen_prefill(case["q"].numpy(), ks, vs, cq, ck, 0.3)
    assert np.array_equal(out, out2)
    # decode of each sequence's last query row over its Lk keys == last prefill row
    last = cq[1:] - 1
    lens = ck[1:] - ck[:-1]
    dec = paged.paged_decode(case["q"].numpy()[last], kc, vc, bt, lens, 0.3)
    np.testing.assert_allclose(dec, out[last], rtol=1e-12)
    # torch CPU baseline path agrees
    ref = sdpa_path.varlen_prefill(case["q"], torch.from_numpy(kc), torch.from_numpy(vc),
                                   case["cu_seqlens_q"], case["cu_seqlens_k"], 0.3,
                                   block_tables=case["block_tables"], compute_dtype=torch.float64)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-9, atol=1e-11)


def test_prefill_rows_subset():
    case = make_prefill_case("cfg3", seed=3, nseq=3, lq=(5, 30), prefix_blocks=(1, 1), bs=16,
                             hq=2, hkv=1, d=8, dtype=torch.float64)
    args = (case["q"].numpy(), case["k_cache"].numpy(), case["v_cache"].numpy(),
            case["cu_seqlens_q"].numpy(), case["cu_seqlens_k"].numpy(), 0.3)
    full = paged.varlen_prefill(*args, block_tables=case["block_tables"].numpy())
    rows = [0, 4, 9, int(case["cu_seqlens_q"][-1]) - 1]
    part = paged.varlen_prefill(*args, block_tables=case["block_tables"].numpy(), rows=rows)
    np.testing.assert_allclose(part[rows], full[rows], rtol=1e-12, atol=1e-14)


def test_fp8_decode_oracle_scales():
    case = make_decode_case("cfg5", seed=1, batch=3, ctx=(40, 300), hq=8, hkv=2, bs=32)
    kc = fp8.decode_e4m3fn(case["k_cache"].view(torch.uint8).numpy())
    vc = fp8.decode_e4m3fn(case["v_cache"].view(torch.uint8).numpy())
    ks, vs = case["k_scale"].numpy(), case["v_scale"].numpy()
    a = paged.paged_decode(case["q"].float().numpy(), kc, vc, case["block_tables"].numpy(),
                           case["context_lens"].numpy(), case["scale"], ks, vs)
    # explicit dequantization gives the same result
    b = paged.paged_decode(case["q"].float().numpy(), kc.astype(np.float64) * ks[None, None, :, None],
                           vc.astype(np.float64) * vs[None, None, :, None], case["block_tables"].numpy(),
                           case["context_lens"].numpy(), case["scale"])
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-13)
    # torch path with in-timed-region dequantization agrees
    c = sdpa_path.paged_decode(case["q"].double(), case["k_cache"], case["v_cache"], case["block_tables"],
                               case["context_lens"], case["scale"], case["k_scale"], case["v_scale"],
                               compute_dtype=torch.float64)
    np.testing.assert_allclose(a, c.numpy(), rtol=1e-6, atol=1e-7)


# ----------------------------------------------------------------- metadata


class _Seq:
    def __init__(self, n, table, cached, sched):
        self.token_ids = list(range(100, 100 + n))
        self.block_table = table
        self.num_cached_tokens = cached
        self.num_scheduled_tokens = sched


def test_prepare_prefill_closed_form_vs_simulation():
    bs = 256
    random.seed(0)
    seqs = []
    for i in range(5):
        n = random.randint(1, 1500)
        table = random.sample(range(40), (n + bs - 1) // bs)
        cached = bs * random.randint(0, (n - 1) // bs) if i % 2 == 0 else 0
        # chunked prefill: schedule a prefix of the remaining tokens
        sched = n - cached if i != 3 else max(1, (n - cached) // 3)
        seqs.append(_Seq(n, table, cached, sched))
    md = metadata.prepare_prefill(seqs, bs)
    # token-by-token simulation
    slots = []
    for s in seqs:
        for pos in range(s.num_cached_tokens, s.num_cached_tokens + s.num_scheduled_tokens):
            slots.append(s.block_table[pos // bs] * bs + pos % bs)
    assert md["slot_mapping"] == slots
    assert md["cu_seqlens_q"][-1] == len(slots)
    assert md["cu_seqlens_k"][1:] == list(np.cumsum([s.num_cached_tokens + s.num_scheduled_tokens
                                                     for s in seqs]))
    has_prefix = any(s.num_cached_tokens for s in seqs)
    assert (md["block_tables"] is not None) == has_prefix


def test_prepare_decode_closed_form():
    bs = 256
    seqs = [_Seq(n, list(range(7, 7 + (n + bs - 1) // bs)), 0, 1) for n in (1, 255, 256, 257, 1000)]
    md = metadata.prepare_decode(seqs, bs, sampled_token_ids=np.arange(50) * 3, batch_slots=[4, 0, 2, 1, 3])
    for s, pos, ctx, slot in zip(seqs, md["positions"], md["context_lens"], md["slot_mapping"]):
        n = len(s.token_ids)
        assert pos == n - 1 and ctx == n
        # the new token's slot is where prepare_prefill would put position n-1
        assert slot == s.block_table[(n - 1) // bs] * bs + (n - 1) % bs
    assert md["input_ids"] == [12, 0, 6, 3, 9]
