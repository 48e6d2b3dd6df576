"""Seeded random sweeps of the attention kernels' shape space on the GPU.

Each case draws its batch, lengths, prefix hits, head counts, head_dim,
block size and dtypes from a fixed seed, runs the reference's step (store
the new K/V, then attend) and checks every output row against
``oracle/sdpa_path`` in float32 on the device (which tests/test_oracle.py
pins against the float64 oracle), with the contract's tolerances.  The
sweeps cover combinations the hand-picked tests do not: prefixes that end
inside a block after a chunked prefill, GQA groups 1 to 8 at head_dim 128
and 256, 16-bit and fp8 caches, block sizes 256 and 512, one to 40
sequences, and decode batches with split-K plans.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle.inputs import make_decode_case, make_prefill_case
from tests.parity import TOL_BF16, TOL_FP8, full_decode_check, full_prefill_check

pytestmark = pytest.mark.gpu


def _prefill_params(seed):
    r = np.random.default_rng(1000 + seed)
    d = int(r.choice([128, 128, 256]))
    hkv = int(r.choice([1, 2, 4, 8]))
    g = int(r.choice([1, 2, 4, 8] if d == 128 else [1, 2, 4]))
    nseq = int(r.integers(1, 41))
    lo = int(r.integers(1, 300))
    hi = lo + int(r.integers(0, 900))
    bs = int(r.choice([256, 512]))
    kv = "fp8" if r.random() < 0.3 else "same"
    dtype = torch.float16 if (kv == "same" and r.random() < 0.3) else torch.bfloat16
    pre = (0, 0) if r.random() < 0.3 else (1, int(r.integers(1, 4)))
    return dict(nseq=nseq, lq=(lo, hi), prefix_blocks=pre, hq=hkv * g, hkv=hkv, d=d, bs=bs, kv=kv, dtype=dtype)


def _chunked_prefix(case, r):
    """Move a random number of each prefixed sequence's first new tokens into
    its prefix (as a chunked prefill leaves them), so prefixes end inside a
    block; the packed layout stays consistent."""
    lq, lk = list(case["lq"]), list(case["lk"])
    keep = []
    for i in range(len(lq)):
        shift = int(r.integers(0, lq[i])) if (case["prefix"][i] > 0 and lq[i] > 1) else 0
        keep.append((shift, lq[i]))
    dev = case["q"].device
    rows, qs = [], 0
    new_lq = []
    for (shift, n) in keep:
        rows.extend(range(qs + shift, qs + n))
        new_lq.append(n - shift)
        qs += n
    idx = torch.tensor(rows, dtype=torch.int64, device=dev)
    for key in ("q", "k_new", "v_new"):
        case[key] = case[key].index_select(0, idx).contiguous()
    case["slot_mapping"] = case["slot_mapping"].index_select(0, idx).contiguous()
    cu_q = np.concatenate([[0], np.cumsum(new_lq)])
    case["lq"] = new_lq
    case["cu_seqlens_q"] = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    case["max_seqlen_q"] = max(new_lq)
    return case


@pytest.mark.parametrize("seed", range(16))
def test_prefill_random_sweep(cuda, seed):
    p = _prefill_params(seed)
    case = make_prefill_case("cfg3", seed=seed, device=cuda, **p)
    r = np.random.default_rng(2000 + seed)
    if case["block_tables"] is not None and r.random() < 0.5:
        # The tokens moved into the prefix were stored by an earlier step:
        # store them now, then drop them from this step's rows.
        kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"], case["slot_mapping"],
                              case["k_scale"], case["v_scale"])
        case = _chunked_prefix(case, r)
    print(f"[sweep] prefill seed={seed} n={case['nseq']} lq={case['lq'][:5]} prefix={case['prefix'][:5]} "
          f"hq={p['hq']} hkv={p['hkv']} d={p['d']} bs={p['bs']} kv={p['kv']} {p['dtype']} "
          f"paged={case['block_tables'] is not None}", flush=True)
    kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"], case["slot_mapping"],
                          case["k_scale"], case["v_scale"])
    if case["block_tables"] is None:
        k, v, ks, vs = case["k_new"], case["v_new"], None, None
    else:
        k, v, ks, vs = case["k_cache"], case["v_cache"], case["k_scale"], case["v_scale"]
    out = kernels.varlen_prefill(case["q"], k, v, case["cu_seqlens_q"], case["cu_seqlens_k"],
                                 case["max_seqlen_q"], case["max_seqlen_k"], case["scale"], causal=True,
                                 block_table=case["block_tables"], k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    tol = TOL_FP8 if p["kv"] == "fp8" else TOL_BF16
    mx, mn = full_prefill_check(case, out, tol)
    print(f"[sweep] prefill seed={seed}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)


def _decode_params(seed):
    r = np.random.default_rng(3000 + seed)
    d = int(r.choice([128, 128, 256]))
    hkv = int(r.choice([1, 2, 4, 8]))
    g = int(r.choice([1, 2, 4, 8, 16] if d == 128 else [1, 2, 4, 8]))
    batch = int(r.integers(1, 65))
    lo = int(r.integers(1, 2000))
    hi = lo + int(r.integers(0, 6000))
    bs = int(r.choice([256, 512]))
    kv = "fp8" if r.random() < 0.3 else "same"
    dtype = torch.float16 if (kv == "same" and r.random() < 0.3) else torch.bfloat16
    return dict(batch=batch, ctx=(lo, hi), hq=hkv * g, hkv=hkv, d=d, bs=bs, kv=kv, dtype=dtype)


@pytest.mark.parametrize("seed", range(16))
def test_decode_random_sweep(cuda, seed):
    p = _decode_params(seed)
    case = make_decode_case("cfg2", seed=seed, device=cuda, amp=1.0, **p)
    print(f"[sweep] decode seed={seed} B={p['batch']} ctx={p['ctx']} hq={p['hq']} hkv={p['hkv']} d={p['d']} "
          f"bs={p['bs']} kv={p['kv']} {p['dtype']}", flush=True)
    kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"], case["slot_mapping"],
                          case["k_scale"], case["v_scale"])
    out = kernels.paged_decode(case["q"], case["k_cache"], case["v_cache"], case["context_lens"],
                               case["block_tables"], case["scale"], k_scale=case["k_scale"],
                               v_scale=case["v_scale"])
    torch.cuda.synchronize()
    tol = TOL_FP8 if p["kv"] == "fp8" else TOL_BF16
    mx, mn = full_decode_check(case, out, tol)
    print(f"[sweep] decode seed={seed}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
