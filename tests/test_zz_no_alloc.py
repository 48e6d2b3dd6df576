"""nq_paged_decode_noalloc (split-K partials in the library's static device
array) against nq_paged_decode with a caller workspace: bit-identical
outputs on two calls in a row, the second with a smaller input, both
through the C ABI.  The entry point has no counterpart in the reference; it
serves callers that cannot allocate."""
import ctypes

import pytest
import torch

from nano_qwen_amd import kernels
from nano_qwen_amd._lib import check, dtype_code, lib, ptr, stream_of
from oracle.inputs import make_decode_case

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # NQ_DECODE_NOALLOC_SCRATCH_BYTES in include/nq_attn.h


def _plan(case):
    W = case["block_tables"].shape[1]
    return kernels.decode_plan(case["batch"], case["hq"], case["hkv"], W, case["block_size"],
                               case["k_cache"].dtype)


def _noalloc(case, out, ns, st):
    q, kc, vc, bt = case["q"], case["k_cache"], case["v_cache"], case["block_tables"]
    fp8 = kc.dtype == torch.float8_e4m3fn
    return lib().nq_paged_decode_noalloc(
        ptr(q), q.stride(0), q.stride(1), ptr(kc), ptr(vc), ptr(bt), bt.stride(0), bt.shape[1],
        ptr(case["context_lens"]), ptr(out), out.stride(0), out.stride(1), case["batch"], case["hq"],
        case["hkv"], case["d"], case["block_size"], kc.shape[0], float(case["scale"]), ns, st,
        dtype_code(q.dtype), dtype_code(kc.dtype), ptr(case["k_scale"]) if fp8 else None,
        ptr(case["v_scale"]) if fp8 else None, stream_of(q))


def _compare(case):
    ns, st = _plan(case)
    print(f"[noalloc] B={case['batch']} Hq={case['hq']} kv={case['k_cache'].dtype} splits={ns} x {st}", flush=True)
    ref = kernels.paged_decode(case["q"], case["k_cache"], case["v_cache"], case["context_lens"],
                               case["block_tables"], case["scale"], case["k_scale"], case["v_scale"])
    out = torch.full_like(ref, float("nan"))
    check(_noalloc(case, out, ns, st), "paged_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "static-scratch decode differs from the workspace decode"
    return ns


def test_noalloc_matches_workspace_decode_twice(cuda):
    big = make_decode_case("cfg4", seed=3, device=cuda, batch=4, ctx=(20000, 32768))
    assert _compare(big) > 1, "the first call must use the split-K scratch"
    # second call, smaller input: the scratch keeps the first call's partials
    small = make_decode_case("cfg2", seed=4, device=cuda, batch=5, ctx=(300, 3000))
    small_ns = _compare(small)
    assert small_ns >= 1


def test_noalloc_fp8_and_single_split(cuda):
    _compare(make_decode_case("cfg5", seed=5, device=cuda, batch=8, ctx=(2000, 8192)))
    _compare(make_decode_case("cfg1", seed=0, device=cuda, dtype=torch.bfloat16))


def test_noalloc_rejects_plans_beyond_the_scratch(cuda):
    case = make_decode_case("cfg2", seed=6, device=cuda, batch=2, ctx=(300, 600))
    d, hq = case["d"], case["hq"]
    # a plan whose partials exceed the static array: rejected before any launch
    per = lib().nq_decode_workspace_bytes(1, hq, d, 64)
    batch = SCRATCH_BYTES // per + 1
    assert lib().nq_decode_workspace_bytes(batch, hq, d, 64) > SCRATCH_BYTES
    q = torch.zeros(batch, hq, d, dtype=torch.bfloat16, device=cuda)
    out = torch.zeros_like(q)
    bt = torch.zeros(batch, 64, dtype=torch.int32, device=cuda)
    ctx = torch.zeros(batch, dtype=torch.int32, device=cuda)
    kc = case["k_cache"]
    rc = lib().nq_paged_decode_noalloc(
        ptr(q), q.stride(0), q.stride(1), ptr(kc), ptr(case["v_cache"]), ptr(bt), 64, 64, ptr(ctx), ptr(out),
        out.stride(0), out.stride(1), batch, hq, case["hkv"], d, 256, kc.shape[0], 0.1, 64, 256,
        dtype_code(q.dtype), dtype_code(kc.dtype), None, None, stream_of(q))
    assert rc == -1
    assert b"scratch" in lib().nq_last_error()


def test_noalloc_plan_grown_past_the_scratch(cuda):
    # fp8 with many query heads: the plan's split count, grown so a caller's
    # workspace would also hold stream-K partials at head_dim 256, sizes more
    # than the static array; the entry point runs with the splits that cover
    # the table and the launch fits its partials in the array.
    case = make_decode_case("cfg5", seed=9, device=cuda, batch=1, ctx=(6000, 8000), hq=128, hkv=8)
    ns, st = _plan(case)
    assert lib().nq_decode_workspace_bytes(1, 128, 256, ns) > SCRATCH_BYTES
    _compare(case)
