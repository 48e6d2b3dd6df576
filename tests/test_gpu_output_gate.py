"""Qwen3.5's output gate on the GPU (models/qwen3_5.py:140-142).

The gated decode store and nq_output_gate against oracle/output_gate.py
applied to the same kernels' ungated output: at most one bf16 ulp, and at
most 0.1% of elements differing (the last float32 bit of exp() may move a
rounding of the sigmoid); also against torch's own eager ops on the GPU.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle.output_gate import output_gate as gate_ref

pytestmark = pytest.mark.gpu


def _ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    def key(t):
        x = t.contiguous().view(torch.int16).cpu().numpy().astype(np.int64)
        return np.where(x < 0, -(x + 32768), x)
    return np.abs(key(a) - key(b))


def _check(got, ref, what):
    u = _ulps(got, ref)
    frac = float((u > 0).mean())
    assert u.max() <= 1 and frac <= 1e-3, f"{what}: max {u.max()} ulp, {frac:.4%} differ"


def _gate_of(n, hq, d, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q_gate = (torch.randn(n, hq, 2 * d, generator=g) * 3).to(torch.bfloat16).to(dev)
    return q_gate[..., d:]     # the gate half of q_proj's output, a strided view


def test_decode_gated_store(cuda):
    """cfg2 (single- and two-split sequences): gated == gate(ungated)."""
    from oracle.inputs import make_decode_case
    c = make_decode_case("cfg2", seed=4, device="cuda")
    B, hq, d = c["q"].shape
    gate = _gate_of(B, hq, d, 1, cuda)
    args = (c["q"].unsqueeze(1), c["k_cache"], c["v_cache"], c["context_lens"], c["block_tables"], c["scale"])
    plain = kernels.paged_decode(*args).squeeze(1)
    gated = kernels.paged_decode(*args, gate=gate).squeeze(1)
    torch.cuda.synchronize()
    ns, _ = kernels.decode_plan(B, hq, c["hkv"], c["block_tables"].shape[1], 256, torch.bfloat16)
    assert ns > 1 and int(c["context_lens"].min()) <= 2048 < int(c["context_lens"].max())
    ref = gate_ref(plain.float().cpu().numpy(), gate.float().cpu().numpy(), "bf16")
    _check(gated, torch.from_numpy(ref).to(torch.bfloat16), "decode gated vs oracle")
    _check(gated, plain * torch.sigmoid(gate), "decode gated vs torch eager")


def test_decode_gated_zero_context_rows(cuda):
    from oracle.inputs import make_decode_case
    c = make_decode_case("cfg2", seed=5, device="cuda")
    c["context_lens"][::7] = 0
    B, hq, d = c["q"].shape
    gate = _gate_of(B, hq, d, 2, cuda)
    out = kernels.paged_decode(c["q"].unsqueeze(1), c["k_cache"], c["v_cache"], c["context_lens"],
                               c["block_tables"], c["scale"], gate=gate).squeeze(1)
    torch.cuda.synchronize()
    assert torch.all(out[::7] == 0)


def test_prefill_gate_pass(cuda):
    """cfg3's full prefill output with the in-place gate pass."""
    from oracle.inputs import make_prefill_case
    c = make_prefill_case("cfg3", seed=6, device="cuda")
    tq, hq, d = c["q"].shape
    gate = _gate_of(tq, hq, d, 3, cuda)
    args = (c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"], c["cu_seqlens_k"], c["max_seqlen_q"],
            c["max_seqlen_k"], c["scale"])
    kernels.store_kvcache(c["k_new"], c["v_new"], c["k_cache"], c["v_cache"], c["slot_mapping"])
    plain = kernels.varlen_prefill(*args, block_table=c["block_tables"])
    gated = kernels.varlen_prefill(*args, block_table=c["block_tables"], gate=gate)
    torch.cuda.synchronize()
    ref = gate_ref(plain.float().cpu().numpy(), gate.float().cpu().numpy(), "bf16")
    _check(gated, torch.from_numpy(ref).to(torch.bfloat16), "prefill gated vs oracle")
    _check(gated, plain * torch.sigmoid(gate), "prefill gated vs torch eager")


def test_output_gate_f16_and_errors(cuda):
    g = torch.Generator().manual_seed(7)
    out = torch.randn(33, 4, 64, generator=g).half().to(cuda)
    gate = torch.randn(33, 4, 64, generator=g).half().to(cuda)
    ref = out * torch.sigmoid(gate)
    kernels.output_gate(out, gate)
    torch.cuda.synchronize()
    d = (out.float() - ref.float()).abs()
    assert float(d.max()) <= float(ref.float().abs().max()) * 2 ** -10
    with pytest.raises(RuntimeError, match="dtype"):
        kernels.output_gate(out.float(), gate.float())


@pytest.mark.parametrize("kind", ["packed", "fp8", "past_list"])
def test_prefill_gated_other_paths(cuda, kind):
    """Packed K/V (no block table), paged fp8 K/V, and a batch whose queues
    outgrow the item list the kernel keeps in LDS (items derived when taken)
    on the persistent kernel's fused store: gated == gate(ungated)."""
    from oracle.inputs import make_prefill_case
    if kind == "packed":
        c = make_prefill_case("cfg3", seed=8, device="cuda", prefix_blocks=(0, 0), lq=(100, 700))
        k, v, bt, ks, vs = c["k_new"], c["v_new"], None, None, None
    elif kind == "past_list":
        c = make_prefill_case("cfg3", seed=13, device="cuda", nseq=300, lq=(1, 300), prefix_blocks=(0, 0))
        assert max(c["lq"]) > 288
        k, v, bt, ks, vs = c["k_new"], c["v_new"], None, None, None
    else:
        c = make_prefill_case("cfg3", seed=9, device="cuda", kv="fp8", lq=(100, 700))
        kernels.store_kvcache(c["k_new"], c["v_new"], c["k_cache"], c["v_cache"], c["slot_mapping"],
                              c["k_scale"], c["v_scale"])
        k, v, bt, ks, vs = c["k_cache"], c["v_cache"], c["block_tables"], c["k_scale"], c["v_scale"]
    tq, hq, d = c["q"].shape
    gate = _gate_of(tq, hq, d, 10, cuda)
    args = (c["q"], k, v, c["cu_seqlens_q"], c["cu_seqlens_k"], c["max_seqlen_q"], c["max_seqlen_k"], c["scale"])
    plain = kernels.varlen_prefill(*args, block_table=bt, k_scale=ks, v_scale=vs)
    gated = kernels.varlen_prefill(*args, block_table=bt, k_scale=ks, v_scale=vs, gate=gate)
    torch.cuda.synchronize()
    ref = gate_ref(plain.float().cpu().numpy(), gate.float().cpu().numpy(), "bf16")
    _check(gated, torch.from_numpy(ref).to(torch.bfloat16), f"prefill {kind} gated vs oracle")


def test_attention_layer_gate(cuda):
    """Attention.forward(q, k, v, gate=...) on a decode step equals the
    kernel-level gated decode."""
    from nano_qwen_amd.layers import Attention
    from nano_qwen_amd.utils.context import reset_context, set_context
    from oracle.inputs import make_decode_case
    c = make_decode_case("cfg2", seed=11, device="cuda")
    B, hq, d = c["q"].shape
    gate = _gate_of(B, hq, d, 12, cuda)
    attn = Attention(hq, d, c["scale"], c["hkv"])
    attn.k_cache, attn.v_cache = c["k_cache"], c["v_cache"]
    set_context(False, slot_mapping=c["slot_mapping"], context_lens=c["context_lens"],
                block_tables=c["block_tables"])
    out = attn(c["q"], c["k_new"], c["v_new"], gate=gate).squeeze(1)
    reset_context()
    ref = kernels.paged_decode(c["q"].unsqueeze(1), c["k_cache"], c["v_cache"], c["context_lens"],
                               c["block_tables"], c["scale"], gate=gate).squeeze(1)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
