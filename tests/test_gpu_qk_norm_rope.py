"""nq_qk_norm_rope_store on the GPU vs oracle/qk_norm_rope.py.

Contract: q_out / k_out bit-exact to the oracle, which fixes the float32
summation order of the mean of squares to the kernel's (any order is a valid
reading of the reference's ``mean``) and rounds every operation on its own;
cache rows bit-exact to what nq_store_kvcache stores for the kernel's own
k_out and the raw v.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle import fp8
from oracle import qk_norm_rope as o

pytestmark = pytest.mark.gpu

NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
INT = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def _ordered(t: torch.Tensor) -> np.ndarray:
    """Bits of a float tensor mapped to integers ordered like the values."""
    bits = t.contiguous().view(INT[t.dtype]).numpy().astype(np.int64)
    top = 1 << (8 * t.element_size() - 1)
    return np.where(bits < 0, -(bits + top), bits)


def assert_ulps(got: torch.Tensor, ref: np.ndarray, what: str):
    ref_t = torch.from_numpy(np.ascontiguousarray(ref, dtype=np.float32)).to(got.dtype)
    assert torch.equal(ref_t.float(), torch.from_numpy(np.asarray(ref, np.float32))) or np.isnan(ref).any()
    g = got.detach().cpu()
    nan_g, nan_r = torch.isnan(g).numpy(), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN pattern differs"
    u = np.abs(_ordered(g) - _ordered(ref_t))[~nan_r]
    frac = float((u > 0).mean()) if u.size else 0.0
    assert u.size == 0 or u.max() == 0, f"{what}: max {u.max()} ulp, {frac:.3%} of elements differ"


def _case(n=97, hq=8, hkv=2, d=128, rot=32, dtype=torch.bfloat16, nb=6, bs=256, max_pos=4096, seed=0):
    g = torch.Generator().manual_seed(seed)
    q_gate = torch.randn(n, hq, 2 * d, generator=g).mul_(2).to(dtype)
    key = torch.randn(n, hkv, d, generator=g).mul_(2).to(dtype)
    val = torch.randn(n, hkv, d, generator=g).to(dtype)
    qw = (torch.rand(d, generator=g) * 2 - 1).to(dtype)
    kw = (torch.rand(d, generator=g) * 2 - 1).to(dtype)
    pos = torch.randint(0, max_pos, (n,), generator=g, dtype=torch.int64)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[::13] = -1
    cs = torch.from_numpy(o.rope_cache(rot, max_pos, 1e7)) if rot else torch.zeros(max_pos, 0)
    kc = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    vc = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    return dict(q_gate=q_gate, key=key, val=val, qw=qw, kw=kw, pos=pos, slots=slots, cs=cs, kc=kc, vc=vc,
                rot=rot, d=d, dtype=dtype)


def _oracle(c, eps=1e-6):
    f = lambda t: t.float().numpy()
    q = f(c["q_gate"])[..., :c["d"]]
    return o.qk_norm_rope(q, f(c["key"]), c["pos"].numpy(), c["cs"].numpy(), c["rot"], f(c["qw"]), f(c["kw"]),
                          eps, NAMES[c["dtype"]])


def _run(c, dev, store=True, eps=1e-6, **kw):
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in c.items()}
    query = g["q_gate"][..., :c["d"]]     # the query half of q_proj's [N, Hq, 2D] output
    q_out, k_out = kernels.qk_norm_rope_store(
        g["pos"], query, g["key"], g["val"], g["qw"], g["kw"], eps, g["cs"], c["rot"],
        k_cache=g["kc"] if store else None, v_cache=g["vc"] if store else None,
        slot_mapping=g["slots"] if store else None, **kw)
    torch.cuda.synchronize()
    return g, q_out, k_out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d,rot", [(128, 32), (128, 128), (128, 0), (256, 64), (64, 16)])
def test_matches_oracle_and_stores(cuda, dtype, d, rot):
    c = _case(d=d, rot=rot, dtype=dtype, seed=d + rot)
    ref_q, ref_k = _oracle(c)
    g, q_out, k_out = _run(c, cuda)
    assert_ulps(q_out, ref_q, "q_out")
    assert_ulps(k_out, ref_k, "k_out")
    # cache rows: the kernel's own k_out and the raw v, bit for bit; other rows untouched
    slots = c["slots"].numpy()
    ok = slots >= 0
    kc, vc = c["kc"].clone(), c["vc"].clone()
    kc.view(-1, *k_out.shape[1:])[torch.from_numpy(slots[ok]).long()] = k_out.cpu()[torch.from_numpy(ok)]
    vc.view(-1, *k_out.shape[1:])[torch.from_numpy(slots[ok]).long()] = c["val"][torch.from_numpy(ok)]
    it = INT[dtype]
    assert torch.equal(g["kc"].cpu().view(it), kc.view(it))
    assert torch.equal(g["vc"].cpu().view(it), vc.view(it))
    # the gate half of q_gate is not written
    assert torch.equal(g["q_gate"][..., d:].cpu().view(it), c["q_gate"][..., d:].view(it))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_cache(cuda, dtype):
    c = _case(dtype=dtype, rot=64, d=256, hq=4, hkv=2, seed=5)
    n, hkv, d = c["key"].shape
    kc8 = torch.zeros(c["kc"].shape, dtype=torch.uint8)
    vc8 = torch.zeros(c["vc"].shape, dtype=torch.uint8)
    k_scale = torch.tensor([0.011, 0.023], dtype=torch.float32)
    v_scale = torch.tensor([0.009, 0.017], dtype=torch.float32)
    c8 = dict(c, kc=kc8.view(torch.float8_e4m3fn), vc=vc8.view(torch.float8_e4m3fn))
    g, q_out, k_out = _run(c8, cuda, k_scale=k_scale.to(cuda), v_scale=v_scale.to(cuda))
    ref_q, ref_k = _oracle(c)
    assert_ulps(q_out, ref_q, "q_out")
    assert_ulps(k_out, ref_k, "k_out")
    kq, vq = kc8.numpy().copy(), vc8.numpy().copy()
    o.store_rows(k_out.cpu().float().numpy(), c["val"].float().numpy(), kq, vq, c["slots"].numpy(),
                 k_scale.numpy(), v_scale.numpy())
    assert np.array_equal(g["kc"].cpu().view(torch.uint8).numpy(), kq)
    assert np.array_equal(g["vc"].cpu().view(torch.uint8).numpy(), vq)


def test_in_place_on_strided_query(cuda):
    """q_out = the query view of q_gate itself and k_out = key: same bits as
    the out-of-place call; the gate half is untouched."""
    c = _case(hq=16, hkv=4, rot=32, seed=9)
    _, q_ref, k_ref = _run(c, cuda)
    g = {k: (v.to(cuda) if torch.is_tensor(v) else v) for k, v in c.items()}
    query = g["q_gate"][..., :128]
    q2, k2 = kernels.qk_norm_rope_store(g["pos"], query, g["key"], g["val"], g["qw"], g["kw"], 1e-6, g["cs"],
                                        32, k_cache=g["kc"], v_cache=g["vc"], slot_mapping=g["slots"],
                                        q_out=query, k_out=g["key"])
    torch.cuda.synchronize()
    assert q2.data_ptr() == query.data_ptr()
    assert torch.equal(q2.cpu().view(torch.int16), q_ref.cpu().view(torch.int16))
    assert torch.equal(k2.cpu().view(torch.int16), k_ref.cpu().view(torch.int16))
    assert torch.equal(g["q_gate"][..., 128:].cpu().view(torch.int16), c["q_gate"][..., 128:].view(torch.int16))


def test_without_cache_empty_and_bad_positions(cuda):
    c = _case(rot=32, seed=11, max_pos=300)
    c["pos"][[0, 5, 50]] = torch.tensor([-1, 300, 10**9])
    ref_q, ref_k = _oracle(c)
    g, q_out, k_out = _run(c, cuda, store=False)
    assert torch.isnan(q_out[[0, 5, 50]].cpu()).all() and torch.isnan(k_out[[0, 5, 50]].cpu()).all()
    assert_ulps(q_out, ref_q, "q_out")
    assert_ulps(k_out, ref_k, "k_out")
    assert torch.equal(g["kc"].cpu().view(torch.int16), c["kc"].view(torch.int16))   # no store
    e = _case(n=0, seed=12)
    _, q0, k0 = _run(e, cuda)
    assert q0.shape[0] == 0 and k0.shape[0] == 0


def test_rejects_bad_arguments(cuda):
    c = _case(rot=24, seed=13)     # rotary_dim not a multiple of 16
    with pytest.raises(RuntimeError, match="rotary_dim"):
        _run(c, cuda)
    c = _case(d=96, rot=32, seed=14)
    with pytest.raises(RuntimeError, match="head_dim"):
        _run(c, cuda)


def test_full_prefill_step(cuda):
    """cfg3's new tokens (about 18.4k, positions prefix + i, the case's slots and
    pool) with Qwen3.5's partial rotary factor 0.25 (R = 32 of D = 128), against
    the oracle; the cache rows hold the kernel's k_out and the raw v."""
    from oracle.inputs import make_norm_rope_case
    c = make_norm_rope_case("cfg3", seed=0, device="cpu")
    d = c["d"]
    f = lambda t: t.float().numpy()
    ref_q, ref_k = o.qk_norm_rope(f(c["q_gate"])[..., :d], f(c["key"]), c["positions"].numpy(),
                                  c["cos_sin_cache"].numpy(), 32, f(c["q_weight"]), f(c["k_weight"]),
                                  c["eps"], "bf16")
    g = {k: (v.to(cuda) if torch.is_tensor(v) else v) for k, v in c.items()}
    q_out, k_out = kernels.qk_norm_rope_store(g["positions"], g["q_gate"][..., :d], g["key"], g["value"],
                                              g["q_weight"], g["k_weight"], c["eps"], g["cos_sin_cache"], 32,
                                              k_cache=g["k_cache"], v_cache=g["v_cache"],
                                              slot_mapping=g["slot_mapping"])
    torch.cuda.synchronize()
    assert_ulps(q_out, ref_q, "q_out")
    assert_ulps(k_out, ref_k, "k_out")
    rows = g["slot_mapping"].long()
    assert torch.equal(g["k_cache"].view(-1, 8, d)[rows].view(torch.int16), k_out.view(torch.int16))
    assert torch.equal(g["v_cache"].view(-1, 8, d)[rows].view(torch.int16), g["value"].view(torch.int16))


class _Norm(torch.nn.Module):
    """Stand-in with the reference GemmaRMSNorm's parameters (layers/layernorm.py)."""

    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w)
        self.eps = eps


class _Rope(torch.nn.Module):
    """Stand-in with InterleavedMRoPE's buffer layout [max_position, 1, R]."""

    def __init__(self, table, rot):
        super().__init__()
        self.rotary_dim = rot
        self.register_buffer("cos_sin_cache", table.unsqueeze(1))


@pytest.mark.parametrize("mode", ["decode", "prefill_paged"])
def test_layer_path_equals_unfused(cuda, mode):
    """layers.qk_norm_rope_store + Attention(kv_stored=True) gives the same bits
    as the unfused sequence: oracle norm + rotation, then Attention.forward
    with its own store (models/qwen3_5.py:135-139)."""
    from nano_qwen_amd.layers import Attention, qk_norm_rope_store
    from nano_qwen_amd.utils.context import reset_context, set_context
    from oracle.inputs import make_norm_rope_case
    name = "cfg2" if mode == "decode" else "cfg3"
    c = make_norm_rope_case(name, seed=3, device="cpu")
    d, hq, hkv = c["d"], c["hq"], c["hkv"]
    if mode == "decode":
        from oracle.inputs import make_decode_case
        base = make_decode_case("cfg2", seed=3, device="cpu")
        ctx = dict(is_prefill=False, slot_mapping=base["slot_mapping"], context_lens=base["context_lens"],
                   block_tables=base["block_tables"])
    else:
        from oracle.inputs import make_prefill_case
        base = make_prefill_case("cfg3", seed=3, device="cpu")
        ctx = dict(is_prefill=True, cu_seqlens_q=base["cu_seqlens_q"], cu_seqlens_k=base["cu_seqlens_k"],
                   max_seqlen_q=base["max_seqlen_q"], max_seqlen_k=base["max_seqlen_k"],
                   slot_mapping=base["slot_mapping"], block_tables=base["block_tables"])
    dev = lambda t: t.to(cuda) if torch.is_tensor(t) else t
    ctx = {k: dev(v) for k, v in ctx.items()}
    outs = []
    for fused in (True, False):
        attn = Attention(hq, d, d ** -0.5, hkv)
        attn.k_cache, attn.v_cache = c["k_cache"].to(cuda), c["v_cache"].to(cuda)
        set_context(**ctx)
        q_gate = c["q_gate"].to(cuda)
        query, key, value = q_gate[..., :d], c["key"].to(cuda), c["value"].to(cuda)
        if fused:
            qn, kn = _Norm(c["q_weight"].to(cuda), c["eps"]), _Norm(c["k_weight"].to(cuda), c["eps"])
            rope = _Rope(c["cos_sin_cache"].to(cuda), c["rotary_dim"])
            q2, k2 = qk_norm_rope_store(c["positions"].to(cuda), query, key, value, qn, kn, rope, attn)
            out = attn(q2, k2, value, kv_stored=True)
        else:
            f = lambda t: t.float().numpy()
            rq, rk = o.qk_norm_rope(f(c["q_gate"])[..., :d], f(c["key"]), c["positions"].numpy(),
                                    c["cos_sin_cache"].numpy(), c["rotary_dim"], f(c["q_weight"]),
                                    f(c["k_weight"]), c["eps"], "bf16")
            q2 = torch.from_numpy(rq).to(torch.bfloat16).to(cuda)
            k2 = torch.from_numpy(rk).to(torch.bfloat16).to(cuda)
            out = attn(q2, k2, value)
        torch.cuda.synchronize()
        outs.append((out.cpu(), attn.k_cache.cpu(), attn.v_cache.cpu()))
        reset_context()
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
