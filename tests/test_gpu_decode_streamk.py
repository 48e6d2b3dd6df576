"""Stream-K paged decode on the GPU (the multi-split path of kernels with one
resident workgroup per CU: fp8 caches, head_dim 256).

The batch's contexts, laid end to end, are cut into equal ranges, one per
workgroup; sequences crossing a range boundary are merged from partials
(csrc/paged_decode.hip; the schedule itself is checked on the CPU in
test_decode_partition.py).  Each case runs with NQ_DECODE_STREAMK=1 and =0
(split-K) and checks every output row against the float32 device reference
(oracle/sdpa_path, pinned against the float64 oracle) and a few rows against
the float64 oracle, at the fp8 tolerance; the two paths must agree with each
other within the same tolerance.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle.inputs import make_decode_case
from oracle.output_gate import output_gate as gate_ref
from tests.parity import TOL_BF16, TOL_FP8, assert_close, decode_reference, f64, full_decode_check, snapshot_decode

pytestmark = pytest.mark.gpu


def _decode(case, gate=None):
    out = kernels.paged_decode(case["q"].unsqueeze(1), case["k_cache"], case["v_cache"], case["context_lens"],
                               case["block_tables"], case["scale"], case["k_scale"], case["v_scale"], gate=gate)
    torch.cuda.synchronize()
    return out


def _schedule(case):
    """The schedule the shim's next decode of ``case`` takes (same plan and
    workspace size as kernels.paged_decode uses)."""
    kc = case["k_cache"]
    B, hq, d = case["batch"], case["q"].shape[1], case["q"].shape[-1]
    hkv, bs, W = kc.shape[2], kc.shape[1], case["block_tables"].shape[1]
    ns, _ = kernels.decode_plan(B, hq, hkv, W, bs, kc.dtype)
    ws = kernels.decode_workspace(kc.device, kernels._lib.lib().nq_decode_workspace_bytes(B, hq, d, ns))
    return kernels.decode_schedule(B, hq, hkv, d, W, bs, kc.dtype, ns, 0 if ws is None else ws.numel())


def _both_paths(case, tol, monkeypatch, oracle_rows=(0,)):
    """Store, then decode on both paths; every row against the device
    reference, ``oracle_rows`` against the float64 oracle (end to end from
    the cache before the store)."""
    rows = [r for r in oracle_rows if int(case["context_lens"][r]) > 0]
    snapshot_decode(case, rows)
    kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"], case["slot_mapping"],
                          case["k_scale"], case["v_scale"])
    torch.cuda.synchronize()
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("NQ_DECODE_STREAMK", mode)
        print(f"[streamk] {case['name']} B={case['batch']} D={case['d']} kv={case['k_cache'].dtype} "
              f"mode={mode}", flush=True)
        # the launch must take the schedule under test, not fall back quietly
        assert _schedule(case) == ("stream-K" if mode == "1" else "split-K")
        out = _decode(case)
        mx, mn = full_decode_check(case, out, tol)
        print(f"[streamk] all rows: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
        outs[mode] = out
    if rows:
        ref = decode_reference(case, rows)
        assert_close(f64(outs["1"][rows, 0]), ref, **tol, what="stream-K vs float64 oracle")
    assert_close(f64(outs["1"]), f64(outs["0"]), **tol, what="stream-K vs split-K")
    return outs


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_streamk_fp8_random_lengths(cuda, seed, monkeypatch):
    # lengths from 0 (padded graph rows) to beyond one range, many sequences
    # crossing range boundaries
    case = make_decode_case("cfg5", seed=seed, device=cuda, batch=48, ctx=(1, 9000))
    ctx = case["context_lens"].clone()
    ctx[[3, 17]] = 0
    ctx[[5, 6]] = 1
    case["context_lens"] = ctx
    slot = case["slot_mapping"].clone()
    slot[[3, 17]] = -1
    for b in (5, 6):  # the new token of a one-token context is position 0
        slot[b] = int(case["block_tables"][b, 0]) * case["block_size"]
    case["slot_mapping"] = slot
    outs = _both_paths(case, TOL_FP8, monkeypatch, oracle_rows=(0, 5, 9))
    for mode in ("1", "0"):
        assert torch.all(outs[mode][[3, 17]] == 0)


def test_streamk_fp8_many_short_sequences(cuda, monkeypatch):
    # short contexts in a wide (padded) table: a multi-split plan whose
    # ranges each hold several whole sequences
    case = make_decode_case("cfg5", seed=7, device=cuda, batch=2000, ctx=(1, 80))
    bt = case["block_tables"]
    wide = torch.full((bt.shape[0], 40), -1, dtype=torch.int32, device=cuda)
    wide[:, :bt.shape[1]] = bt
    case["block_tables"] = wide
    _both_paths(case, TOL_FP8, monkeypatch, oracle_rows=(0, 999, 1999))


@pytest.mark.parametrize("kv", ["same", "fp8"])
def test_streamk_head_dim_256(cuda, kv, monkeypatch):
    case = make_decode_case("cfg5", seed=11, device=cuda, batch=24, ctx=(1, 6000), d=256, hq=32, hkv=8, kv=kv)
    _both_paths(case, TOL_FP8 if kv == "fp8" else TOL_BF16, monkeypatch, oracle_rows=(0, 1))


def test_streamk_gated(cuda, monkeypatch):
    """The gate in the stream-K stores (whole sequences) and merge (the rest)."""
    case = make_decode_case("cfg5", seed=12, device=cuda, batch=40, ctx=(1, 9000))
    B, hq, d = case["batch"], case["hq"], case["d"]
    g = torch.Generator().manual_seed(3)
    gate = (torch.randn(B, hq, 2 * d, generator=g) * 3).to(torch.bfloat16).to(cuda)[..., d:]
    monkeypatch.setenv("NQ_DECODE_STREAMK", "1")
    assert _schedule(case) == "stream-K"
    plain = _decode(case).squeeze(1)
    gated = _decode(case, gate=gate).squeeze(1)
    ref = torch.from_numpy(gate_ref(plain.float().cpu().numpy(), gate.float().cpu().numpy(), "bf16"))
    ref = ref.to(torch.bfloat16)
    a = gated.contiguous().view(torch.int16).cpu().numpy().astype(np.int64)
    b = ref.contiguous().view(torch.int16).cpu().numpy().astype(np.int64)
    ulps = np.abs(np.where(a < 0, -(a + 32768), a) - np.where(b < 0, -(b + 32768), b))
    assert ulps.max() <= 1 and float((ulps > 0).mean()) <= 1e-3, f"max {ulps.max()} ulp"


def test_streamk_graph_replay(cuda, monkeypatch):
    """Captured once, replayed with new context lengths: the ranges are
    recomputed on the device from context_lens at every replay."""
    monkeypatch.setenv("NQ_DECODE_STREAMK", "1")
    case = make_decode_case("cfg5", seed=13, device=cuda, batch=32, ctx=(2000, 8000))
    q = case["q"].unsqueeze(1)
    ctx = case["context_lens"]
    out = torch.empty(case["batch"], 1, case["hq"], case["d"], dtype=q.dtype, device=cuda)

    def step():
        kernels.paged_decode(q, case["k_cache"], case["v_cache"], ctx, case["block_tables"], case["scale"],
                             case["k_scale"], case["v_scale"], out=out)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        step()
        assert _schedule(case) == "stream-K"
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    gen = torch.Generator().manual_seed(5)
    orig = case["context_lens"].cpu()
    for rep in range(3):
        # at most each row's original length: its table holds those blocks
        new = (torch.rand(case["batch"], generator=gen) * orig).to(torch.int32).clamp_(min=1)
        new[rep] = 0
        ctx.copy_(new.to(torch.int32))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        step()
        torch.cuda.synchronize()
        assert torch.equal(replayed, out), f"replay {rep} differs from the eager call"
        full_decode_check(dict(case, context_lens=ctx), out, TOL_FP8)
