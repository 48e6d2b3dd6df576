"""The decode step in one launch (nq_paged_decode_store): the new token's KV
store and the paged decode (layers/attention.py:62-63 then :71-74).

For slot mappings that follow the decode contract (slot of token ctx - 1, or
-1), the fused call must leave exactly the cache bytes nq_store_kvcache
leaves and produce exactly the output of nq_store_kvcache followed by
nq_paged_decode -- bit for bit, on the split-K and stream-K schedules, one-
and multi-split rows, 0-token rows, skipped slots, fp8 caches fed bf16 and
f32 rows, head_dim 256 and the output gate.  Every row is also checked
against the float32 device reference.
"""
import pytest
import torch

from nano_qwen_amd import kernels
from oracle.inputs import make_decode_case
from tests.parity import TOL_BF16, TOL_FP8, full_decode_check

pytestmark = pytest.mark.gpu


def _two_calls(case, k_new, v_new, gate=None):
    kc, vc = case["k_cache"].clone(), case["v_cache"].clone()
    kernels.store_kvcache(k_new, v_new, kc, vc, case["slot_mapping"], case["k_scale"], case["v_scale"])
    out = kernels.paged_decode(case["q"].unsqueeze(1), kc, vc, case["context_lens"], case["block_tables"],
                               case["scale"], case["k_scale"], case["v_scale"], gate=gate)
    torch.cuda.synchronize()
    return out, kc, vc


def _fused(case, k_new, v_new, gate=None):
    kc, vc = case["k_cache"].clone(), case["v_cache"].clone()
    out = kernels.paged_decode(case["q"].unsqueeze(1), kc, vc, case["context_lens"], case["block_tables"],
                               case["scale"], case["k_scale"], case["v_scale"], gate=gate,
                               k=k_new, v=v_new, slot_mapping=case["slot_mapping"])
    torch.cuda.synchronize()
    return out, kc, vc


def _edge_rows(case, cuda):
    """Rows 1 and 2: 0-token graph padding (slot -1); row 3: a skipped store
    on a live row (its attention reads the cache as it is); row 4: one
    token."""
    ctx, slot = case["context_lens"].clone(), case["slot_mapping"].clone()
    B = case["batch"]
    if B > 4:
        ctx[[1, 2]] = 0
        slot[[1, 2]] = -1
        slot[3] = -1
        ctx[4] = 1
        slot[4] = int(case["block_tables"][4, 0]) * case["block_size"]
    case["context_lens"], case["slot_mapping"] = ctx, slot


def _check(case, k_new, v_new, tol, gate=None, mode=None, monkeypatch=None):
    if mode is not None:
        monkeypatch.setenv("NQ_DECODE_STREAMK", mode)
    print(f"[decode_store] {case['name']} B={case['batch']} D={case['d']} kv={case['k_cache'].dtype} "
          f"new={k_new.dtype} mode={mode} gate={gate is not None}", flush=True)
    o2, k2, v2 = _two_calls(case, k_new, v_new, gate)
    o1, k1, v1 = _fused(case, k_new, v_new, gate)
    assert torch.equal(k1.view(torch.uint8), k2.view(torch.uint8)), "K cache bytes differ from nq_store_kvcache"
    assert torch.equal(v1.view(torch.uint8), v2.view(torch.uint8)), "V cache bytes differ from nq_store_kvcache"
    assert torch.equal(o1, o2), "fused output differs from store + decode"
    if gate is None:
        full_decode_check(dict(case, k_cache=k1, v_cache=v1), o1, tol)
    return o1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_store_bf16_f16(cuda, dtype):
    case = make_decode_case("cfg2", seed=3, device=cuda, batch=40, ctx=(1, 5000), dtype=dtype)
    _edge_rows(case, cuda)
    _check(case, case["k_new"], case["v_new"], TOL_BF16)


@pytest.mark.parametrize("mode", ["1", "0"])
@pytest.mark.parametrize("new", ["bf16", "f32"])
def test_fused_store_fp8(cuda, mode, new, monkeypatch):
    case = make_decode_case("cfg5", seed=4, device=cuda, batch=48, ctx=(1, 9000))
    _edge_rows(case, cuda)
    k_new, v_new = case["k_new"], case["v_new"]
    if new == "f32":
        k_new, v_new = k_new.float() * 1.37, v_new.float() * 0.71  # values between bf16 codes, some saturate
    _check(case, k_new, v_new, TOL_FP8, mode=mode, monkeypatch=monkeypatch)


@pytest.mark.parametrize("kv", ["same", "fp8"])
def test_fused_store_head_dim_256(cuda, kv):
    case = make_decode_case("cfg5", seed=5, device=cuda, batch=20, ctx=(1, 6000), d=256, hq=16, hkv=4, kv=kv)
    _edge_rows(case, cuda)
    _check(case, case["k_new"], case["v_new"], TOL_FP8 if kv == "fp8" else TOL_BF16)


def test_fused_store_gated_and_long_split(cuda):
    case = make_decode_case("cfg4", seed=6, device=cuda, batch=4, ctx=(20000, 32768))
    B, hq, d = case["batch"], case["hq"], case["d"]
    g = torch.Generator().manual_seed(9)
    gate = (torch.randn(B, hq, 2 * d, generator=g) * 3).to(torch.bfloat16).to(cuda)[..., d:]
    _check(case, case["k_new"], case["v_new"], TOL_BF16, gate=gate)


def test_fused_store_strided_rows_and_errors(cuda):
    # k/v as views into a wider [B, 3 * Hkv, D] projection output
    case = make_decode_case("cfg2", seed=7, device=cuda, batch=6, ctx=(100, 3000))
    B, hkv, d = case["batch"], case["hkv"], case["d"]
    qkv = torch.randn(B, 3 * hkv, d, dtype=torch.bfloat16, device=cuda)
    k_new, v_new = qkv[:, hkv:2 * hkv], qkv[:, 2 * hkv:]
    _check(case, k_new, v_new, TOL_BF16)
    with pytest.raises(RuntimeError, match="dtype"):
        kernels.paged_decode(case["q"].unsqueeze(1), case["k_cache"], case["v_cache"], case["context_lens"],
                             case["block_tables"], case["scale"], k=k_new.half(), v=v_new.half(),
                             slot_mapping=case["slot_mapping"])
