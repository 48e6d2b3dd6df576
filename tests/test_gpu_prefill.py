"""Causal varlen prefill on the GPU vs the float64 oracle (layers/attention.py:64-70).

Each case runs the reference's prefill step: store the new K/V through
slot_mapping, then attend -- over the packed new K/V when no sequence has a
prefix-cache hit, otherwise over the whole paged cache through block_tables.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle.inputs import make_prefill_case
from tests.parity import (TOL_BF16, TOL_FP8, assert_close, f64, full_prefill_check, prefill_reference,
                          snapshot_prefill)

pytestmark = pytest.mark.gpu


def run_step(case):
    kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"],
                          case["slot_mapping"], case["k_scale"], case["v_scale"])
    if case["block_tables"] is None:
        k, v, ks, vs = case["k_new"], case["v_new"], None, None
    else:
        k, v, ks, vs = case["k_cache"], case["v_cache"], case["k_scale"], case["v_scale"]
    out = kernels.varlen_prefill(case["q"], k, v, case["cu_seqlens_q"], case["cu_seqlens_k"],
                                 case["max_seqlen_q"], case["max_seqlen_k"], case["scale"], causal=True,
                                 block_table=case["block_tables"], k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    return out


def check(case, seq_ids, tol, rows_per_seq=None, all_rows=False):
    """The float64 oracle on ``seq_ids`` (``rows_per_seq`` sampled rows each);
    with ``all_rows`` also every output row against the float32 device
    reference."""
    print(f"[prefill] {case['name']} n={case['nseq']} lq={case['lq'][:6]} prefix={case['prefix'][:6]} "
          f"kv={case['k_cache'].dtype} paged={case['block_tables'] is not None}", flush=True)
    snapshot_prefill(case, seq_ids)
    out = run_step(case)
    assert out.shape == case["q"].shape
    rows, ref = prefill_reference(case, seq_ids, rows_per_seq)
    res = assert_close(f64(out[torch.from_numpy(rows).to(out.device)]), ref, **tol, what=case["name"])
    if all_rows:
        mx, mn = full_prefill_check(case, out, tol)
        print(f"[prefill] {case['name']} all {out.shape[0]} rows: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    return res


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_packed_no_prefix(cuda, dtype):
    case = make_prefill_case("cfg3", seed=0, device=cuda, nseq=5, lq=(1, 400), prefix_blocks=(0, 0),
                             dtype=dtype)
    assert case["block_tables"] is None
    check(case, range(5), TOL_BF16)


def test_prefill_packed_tile_edges(cuda):
    case = make_prefill_case("cfg3", seed=1, device=cuda, nseq=8, lq=(1, 1), prefix_blocks=(0, 0))
    # replace lengths by tile-boundary values and rebuild the packed metadata
    lens = [1, 2, 63, 64, 65, 127, 128, 129]
    tot = sum(lens)
    g = torch.Generator(device=cuda).manual_seed(3)
    case["q"] = torch.randn(tot, 32, 128, generator=g, device=cuda).to(torch.bfloat16)
    case["k_new"] = torch.randn(tot, 8, 128, generator=g, device=cuda).to(torch.bfloat16)
    case["v_new"] = torch.randn(tot, 8, 128, generator=g, device=cuda).to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=cuda)
    case.update(lq=lens, lk=lens, prefix=[0] * 8, cu_seqlens_q=cu, cu_seqlens_k=cu,
                max_seqlen_q=max(lens), max_seqlen_k=max(lens),
                slot_mapping=torch.full((tot,), -1, dtype=torch.int32, device=cuda))
    check(case, range(8), TOL_BF16)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prefill_paged_prefix(cuda, seed):
    case = make_prefill_case("cfg3", seed=seed, device=cuda, nseq=4, lq=(1, 700), prefix_blocks=(1, 3))
    assert case["block_tables"] is not None
    check(case, range(4), TOL_BF16)


def test_prefill_chunked_unaligned_prefix(cuda):
    """A chunked prefill leaves num_cached_tokens off block boundaries
    (scheduler/scheduler.py:47-51): P = Lk - Lq need not be a multiple of 256."""
    case = make_prefill_case("cfg3", seed=4, device=cuda, nseq=3, lq=(50, 300), prefix_blocks=(1, 2))
    bs = 256
    pre = [37, 0, 300]
    lq = case["lq"]
    lk = [p + q for p, q in zip(pre, lq)]
    nb = case["num_blocks"]
    need = sum((x + bs - 1) // bs for x in lk)
    assert need <= nb
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(2))
    W = max((x + bs - 1) // bs for x in lk)
    bt = torch.full((3, W), -1, dtype=torch.int32)
    off = 0
    slots = []
    for i in range(3):
        n = (lk[i] + bs - 1) // bs
        bt[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
        slots += [int(bt[i, p // bs]) * bs + p % bs for p in range(pre[i], lk[i])]
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device=cuda)
    case.update(prefix=pre, lk=lk, cu_seqlens_k=cu_k, max_seqlen_k=max(lk), block_tables=bt.to(cuda),
                slot_mapping=torch.tensor(slots, dtype=torch.int32, device=cuda))
    check(case, range(3), TOL_BF16)


def test_prefill_group_sizes(cuda):
    for G, hkv in ((1, 4), (2, 4), (8, 2), (16, 1)):
        case = make_prefill_case("cfg3", seed=5, device=cuda, nseq=3, lq=(20, 300), prefix_blocks=(1, 1),
                                 hq=G * hkv, hkv=hkv)
        check(case, range(3), TOL_BF16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_fp8_paged(cuda, dtype):
    case = make_prefill_case("cfg3", seed=6, device=cuda, nseq=4, lq=(1, 600), prefix_blocks=(1, 2),
                             kv="fp8", dtype=dtype)
    check(case, range(4), TOL_FP8)


def test_prefill_fp8_group_sizes(cuda):
    """fp8 K/V on the persistent kernel at GQA groups 1, 2, 8 and 16: each
    item takes the K and V scales of its own kv head."""
    for G, hkv in ((1, 4), (2, 4), (8, 2), (16, 1)):
        case = make_prefill_case("cfg3", seed=12, device=cuda, nseq=3, lq=(20, 300), prefix_blocks=(1, 1),
                                 hq=G * hkv, hkv=hkv, kv="fp8")
        check(case, range(3), TOL_FP8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_fp8_packed(cuda, dtype):
    """fp8 K/V packed by cu_seqlens_k (no block table), partial last tiles
    included: against the float32 reference over the dequantized codes."""
    from oracle import sdpa_path
    from oracle.inputs import fp8_scales, quantize_fp8_torch
    case = make_prefill_case("cfg3", seed=13, device=cuda, nseq=5, lq=(1, 500), prefix_blocks=(0, 0), dtype=dtype)
    k, v = case["k_new"], case["v_new"]
    ks, vs = fp8_scales(k) * 1.5, fp8_scales(v) * 0.75   # 0.75: the largest values saturate at 448
    k8, v8 = quantize_fp8_torch(k, ks), quantize_fp8_torch(v, vs)
    out = kernels.varlen_prefill(case["q"], k8, v8, case["cu_seqlens_q"], case["cu_seqlens_k"], case["max_seqlen_q"],
                                 case["max_seqlen_k"], case["scale"], causal=True, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kd = k8.float() * ks.view(1, -1, 1)
    vd = v8.float() * vs.view(1, -1, 1)
    ref = sdpa_path.varlen_prefill(case["q"].float(), kd, vd, case["cu_seqlens_q"], case["cu_seqlens_k"],
                                   case["scale"])
    assert_close(f64(out), f64(ref), **TOL_FP8, what="fp8 packed")


def test_decode_equals_last_prefill_row(cuda):
    """Cross-kernel invariant: the decode output of a sequence equals the last
    row of the causal prefill over the same keys."""
    case = make_prefill_case("cfg3", seed=7, device=cuda, nseq=4, lq=(5, 900), prefix_blocks=(1, 2))
    out = run_step(case)
    last = (case["cu_seqlens_q"][1:] - 1).long()
    lk = torch.tensor(case["lk"], dtype=torch.int32, device=cuda)
    dec = kernels.paged_decode(case["q"][last].unsqueeze(1), case["k_cache"], case["v_cache"], lk,
                               case["block_tables"], case["scale"])
    torch.cuda.synchronize()
    assert_close(f64(dec[:, 0]), f64(out[last]), max_abs=1e-2, mean_abs=1e-3, what="decode vs prefill last row")


@pytest.mark.slow
def test_prefill_cfg3_full(cuda):
    case = make_prefill_case("cfg3", seed=0, device=cuda)
    check(case, list(range(16)), TOL_BF16, rows_per_seq=24, all_rows=True)


@pytest.mark.slow
def test_prefill_cfg3_full_fp8(cuda):
    """cfg3's sequences over an fp8 cache: every output row against the
    float32 device reference over the dequantized cache."""
    case = make_prefill_case("cfg3", seed=0, device=cuda, kv="fp8")
    check(case, [0, 3, 8], TOL_FP8, rows_per_seq=24, all_rows=True)


def test_prefill_queue_resets_between_calls(cuda):
    """The persistent kernel's work-queue counters come back to zero after
    every call: repeated calls (different shapes in between) give bitwise
    identical outputs, and the workspace reads zero afterwards."""
    big = make_prefill_case("cfg3", seed=8, device=cuda, nseq=6, lq=(100, 900), prefix_blocks=(1, 2))
    small = make_prefill_case("cfg3", seed=9, device=cuda, nseq=1, lq=(30, 30), prefix_blocks=(0, 0),
                              hq=8, hkv=2)
    first = run_step(big).clone()
    for _ in range(3):
        run_step(small)
        again = run_step(big)
        assert torch.equal(first, again)
    ws = kernels.prefill_workspace(cuda)
    assert int(ws.abs().sum()) == 0


def test_prefill_many_sequences_cost_order(cuda):
    """70 sequences: the list of each queue's items, built at launch, spans
    two 64-sequence steps of the wave scan (and every lane row of it)."""
    case = make_prefill_case("cfg3", seed=10, device=cuda, nseq=70, lq=(1, 160), prefix_blocks=(1, 1))
    check(case, range(70), TOL_BF16)


@pytest.mark.parametrize("kind", ["d128", "d256", "fp8"])
def test_prefill_cost_order_past_item_list(cuda, kind):
    """Queues whose bound (kv-head groups x query tiles) outgrows the item
    list the kernel keeps in LDS (1984 items at head_dim 128: 300 sequences
    of up to 300 rows bound each queue at 300 x 10; 4096 at 256: 1000 x 10 /
    2) take the cost order derived item by item (the kernels built without
    the list), across several 64-sequence steps of its select."""
    nseq = 1000 if kind == "d256" else 300
    extra = dict(d=256, hq=16, hkv=4) if kind == "d256" else dict(kv="fp8") if kind == "fp8" else {}
    case = make_prefill_case("cfg3", seed=12, device=cuda, nseq=nseq, lq=(1, 300), prefix_blocks=(0, 1), **extra)
    assert max(case["lq"]) > 288  # 10 query tiles of 32 rows
    check(case, range(0, nseq, 37 if kind == "d256" else 11), TOL_FP8 if kind == "fp8" else TOL_BF16)


def test_prefill_query_tile_order_past_lds_bounds(cuda):
    """1100 sequences exceed the sequence bounds the kernel keeps in LDS, so
    its queue runs in query-tile order (items without rows included)."""
    case = make_prefill_case("cfg3", seed=11, device=cuda, nseq=1100, lq=(1, 40), prefix_blocks=(0, 0),
                             hq=8, hkv=2)
    assert case["block_tables"] is None
    check(case, range(0, 1100, 7), TOL_BF16)


@pytest.mark.parametrize("kind", ["packed", "paged", "fp8", "f16_group8"])
def test_prefill_head_dim_256(cuda, kind):
    """head_dim 256, the reference model's own full-attention layers
    (models/qwen3_5.py:69-72 with the transformers default): packed and paged
    K/V, fp8 K/V, and f16 with a GQA group of 8."""
    kw = dict(nseq=4, lq=(1, 600), d=256, hq=16, hkv=4)
    if kind == "packed":
        case = make_prefill_case("cfg3", seed=20, device=cuda, prefix_blocks=(0, 0), **kw)
    elif kind == "paged":
        case = make_prefill_case("cfg3", seed=21, device=cuda, prefix_blocks=(1, 3), **kw)
    elif kind == "fp8":
        case = make_prefill_case("cfg3", seed=22, device=cuda, prefix_blocks=(1, 2), kv="fp8", **kw)
    else:
        kw.update(hq=16, hkv=2)
        case = make_prefill_case("cfg3", seed=23, device=cuda, prefix_blocks=(1, 2), dtype=torch.float16, **kw)
    check(case, range(4), TOL_FP8 if kind == "fp8" else TOL_BF16)


def test_prefill_head_dim_256_gated(cuda):
    """The output gate at head_dim 256 (in the persistent kernel's output store, launch shape D)."""
    from oracle.output_gate import output_gate as gate_ref
    case = make_prefill_case("cfg3", seed=24, device=cuda, nseq=3, lq=(50, 500), prefix_blocks=(1, 2),
                             d=256, hq=16, hkv=4)
    run_step(case)
    tq, hq, d = case["q"].shape
    g = torch.Generator().manual_seed(5)
    gate = (torch.randn(tq, hq, 2 * d, generator=g) * 3).to(torch.bfloat16).to(cuda)[..., d:]
    args = (case["q"], case["k_cache"], case["v_cache"], case["cu_seqlens_q"], case["cu_seqlens_k"],
            case["max_seqlen_q"], case["max_seqlen_k"], case["scale"])
    plain = kernels.varlen_prefill(*args, block_table=case["block_tables"])
    gated = kernels.varlen_prefill(*args, block_table=case["block_tables"], gate=gate)
    torch.cuda.synchronize()
    ref = torch.from_numpy(gate_ref(plain.float().cpu().numpy(), gate.float().cpu().numpy(), "bf16"))
    diff = (gated.cpu().view(torch.int16).int() - ref.to(torch.bfloat16).view(torch.int16).int()).abs()
    assert int(diff.max()) <= 1 and float((diff > 0).float().mean()) <= 1e-3


def test_prefill_two_streams_own_queues(cuda):
    """Launches on two streams at once use their own work-queue counters:
    both outputs equal the single-stream results, and both streams' counters
    read zero afterwards."""
    a = make_prefill_case("cfg3", seed=40, device=cuda, nseq=5, lq=(200, 900), prefix_blocks=(1, 2))
    b = make_prefill_case("cfg3", seed=41, device=cuda, nseq=3, lq=(100, 700), prefix_blocks=(0, 0))
    ra, rb = run_step(a).clone(), run_step(b).clone()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
    outs = {}
    for rep in range(3):
        with torch.cuda.stream(s1):
            outs["a"] = run_step_async(a)
            q1 = kernels.prefill_workspace(cuda)
        with torch.cuda.stream(s2):
            outs["b"] = run_step_async(b)
            q2 = kernels.prefill_workspace(cuda)
        assert q1.data_ptr() != q2.data_ptr()
        torch.cuda.synchronize()
        assert torch.equal(outs["a"], ra) and torch.equal(outs["b"], rb), f"rep {rep}"
        assert int(q1.count_nonzero()) == 0 and int(q2.count_nonzero()) == 0


def run_step_async(case):
    """The attention call of run_step (K/V already stored), without a sync."""
    if case["block_tables"] is None:
        k, v, ks, vs = case["k_new"], case["v_new"], None, None
    else:
        k, v, ks, vs = case["k_cache"], case["v_cache"], case["k_scale"], case["v_scale"]
    return kernels.varlen_prefill(case["q"], k, v, case["cu_seqlens_q"], case["cu_seqlens_k"],
                                  case["max_seqlen_q"], case["max_seqlen_k"], case["scale"], causal=True,
                                  block_table=case["block_tables"], k_scale=ks, v_scale=vs)


def test_prefill_queue_debug_check(cuda, monkeypatch):
    """NQ_DEBUG_PREFILL_QUEUE makes every prefill verify on the host that
    the launch left its work-queue counters at zero."""
    monkeypatch.setattr(kernels, "_DEBUG_QUEUE", True)
    case = make_prefill_case("cfg3", seed=42, device=cuda, nseq=3, lq=(50, 400), prefix_blocks=(1, 1))
    check(case, range(3), TOL_BF16)


