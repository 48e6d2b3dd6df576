"""nq_gdn_decode on the GPU vs oracle/gdn.py (float64).

Contract (floating point; FlashInfer's rounding is not pinned): the state,
kept in float32, within 2e-5 of the float64 state relative to its largest
entry; the output within 1 bf16 (or f16) ulp of the float64 value plus 1e-3 of
the largest output.  Skipped sequences leave their output and every other
slot untouched.
"""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from oracle import gdn

pytestmark = pytest.mark.gpu


def _case(B=6, H=4, HV=8, slots=10, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 128, generator=g).to(dtype)
    k = torch.randn(B, H, 128, generator=g).to(dtype)
    v = torch.randn(B, HV, 128, generator=g).to(dtype)
    a = torch.randn(B, HV, generator=g).to(dtype)
    b = torch.randn(B, HV, generator=g).to(dtype)
    A_log = torch.randn(HV, generator=g) * 0.5
    dt = torch.randn(HV, generator=g) * 0.5
    state = torch.randn(slots, HV, 128, 128, generator=g) * 0.05
    idx = torch.randperm(slots, generator=g)[:B].to(torch.int32)
    idx[1] = -1
    return dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt=dt, state=state, idx=idx)


def _ref(c, state):
    f = lambda t: t.double().numpy()
    return gdn.gdn_decode(f(c["q"]), f(c["k"]), f(c["v"]), f(c["a"]), f(c["b"]), f(c["A_log"]), f(c["dt"]),
                          state, c["idx"].numpy())


def _run(c, dev, state_dev, out=None):
    g = {k: v.to(dev) for k, v in c.items() if k != "state"}
    o = kernels.gdn_decode(g["q"], g["k"], g["v"], g["a"], g["b"], g["A_log"], g["dt"], state_dev, g["idx"], out=out)
    torch.cuda.synchronize()
    return o


def _check(c, out, ref, state_dev, ref_state, live):
    tol_ulp = 2 ** -8 if out.dtype == torch.bfloat16 else 2 ** -11
    o = out.float().cpu().numpy()[live]
    r = ref[live]
    assert np.all(np.abs(o - r) <= tol_ulp * np.abs(r) + 1e-3 * np.abs(r).max()), float(np.abs(o - r).max())
    s = state_dev.cpu().double().numpy()
    assert np.abs(s - ref_state).max() <= 2e-5 * np.abs(ref_state).max()


def _prefill_close(out, ref, state, ref_state):
    """Chunked prefill against the exact recurrence: the kernel's products
    take 16-bit operands (rounded unit keys and queries, the state, the
    inverse, the updates) with float32 accumulation, as the reference's
    Triton chunk kernels do, so errors are a few 16-bit ulps of the largest
    values, not of each element: max within 2% and mean within 0.1% of the
    largest reference magnitude, for the outputs and for the final states."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    s = np.asarray(state, dtype=np.float64)
    rs = np.asarray(ref_state, dtype=np.float64)
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(s))
    om, sm = np.abs(r).max(), np.abs(rs).max()
    eo, es = np.abs(o - r), np.abs(s - rs)
    assert eo.max() <= 2e-2 * om and eo.mean() <= 1e-3 * om, (float(eo.max()), float(eo.mean()), float(om))
    assert es.max() <= 2e-2 * sm and es.mean() <= 1e-3 * sm, (float(es.max()), float(es.mean()), float(sm))
    return float(eo.max() / om), float(es.max() / sm)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gdn_decode_matches_oracle(cuda, dtype):
    c = _case(dtype=dtype, seed=1)
    state_dev = c["state"].clone().to(cuda)
    sentinel = torch.full((6, 8, 128), 7.0, dtype=dtype, device=cuda)
    out = _run(c, cuda, state_dev, out=sentinel)
    ref_state = c["state"].double().numpy()
    ref = _ref(c, ref_state)
    live = c["idx"].numpy() >= 0
    _check(c, out, ref, state_dev, ref_state, live)
    assert torch.all(out[1] == 7.0)   # the skipped sequence's row is not written


def test_gdn_decode_sequence_of_steps(cuda):
    """Ten decode steps on the same slots: the recurrence stays on the float64
    trajectory (the state carries every step's rounding forward)."""
    c = _case(B=3, H=2, HV=4, slots=4, seed=2)
    c["idx"] = torch.tensor([3, 0, 2], dtype=torch.int32)
    state_dev = c["state"].clone().to(cuda)
    ref_state = c["state"].double().numpy()
    g = torch.Generator().manual_seed(3)
    for step in range(10):
        for key in ("q", "k", "v", "a", "b"):
            c[key] = torch.randn(c[key].shape, generator=g).to(torch.bfloat16)
        out = _run(c, cuda, state_dev)
        ref = _ref(c, ref_state)
        _check(c, out, ref, state_dev, ref_state, np.ones(3, bool))


def test_gdn_decode_delta_rule_property(cuda):
    """No decay, beta = 1: after the step, S k = v for the step's key (the
    defining property of the delta rule), on the GPU state."""
    c = _case(B=2, H=1, HV=2, slots=2, seed=4)
    c["idx"] = torch.tensor([0, 1], dtype=torch.int32)
    c["A_log"][:] = -80.0
    c["b"][:] = 60.0
    state_dev = c["state"].clone().to(cuda)
    _run(c, cuda, state_dev)
    S = state_dev.cpu().double().numpy()
    for bi in range(2):
        kn = gdn.l2norm(c["k"][bi, 0].double().numpy())
        for hv in range(2):
            np.testing.assert_allclose(S[bi, hv] @ kn, c["v"][bi, hv].double().numpy(), atol=2e-4)


def test_gdn_decode_rejects(cuda):
    c = _case(seed=5)
    state_dev = c["state"].clone().to(cuda)
    with pytest.raises(RuntimeError):
        kernels.gdn_decode(c["q"].to(cuda), c["k"].to(cuda), c["v"].to(cuda), c["a"].to(cuda), c["b"].to(cuda),
                           c["A_log"].to(cuda), c["dt"].to(cuda), state_dev.double(), c["idx"].to(cuda))


@pytest.mark.parametrize("from_slot", [False, True])
def test_gdn_prefill_matches_oracle(cuda, from_slot):
    """Packed sequences of lengths 1 .. 300 (incl. a tail not a multiple of the
    prefetch depth), zero or pooled initial state, one skipped slot."""
    g = torch.Generator().manual_seed(6)
    lens = [1, 5, 37, 300, 4]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T, H, HV = int(cu[-1]), 2, 4
    bf = torch.bfloat16
    q, k = torch.randn(T, H, 128, generator=g).to(bf), torch.randn(T, H, 128, generator=g).to(bf)
    v = torch.randn(T, HV, 128, generator=g).to(bf)
    a, b = torch.randn(T, HV, generator=g).to(bf), torch.randn(T, HV, generator=g).to(bf)
    A_log, dt = torch.randn(HV, generator=g) * 0.5, torch.randn(HV, generator=g) * 0.5
    state = torch.randn(8, HV, 128, 128, generator=g) * 0.05
    idx = torch.tensor([6, 0, -1, 3, 5], dtype=torch.int32)
    state_dev = state.clone().to(cuda)
    out = kernels.gdn_prefill(q.to(cuda), k.to(cuda), v.to(cuda), a.to(cuda), b.to(cuda), A_log.to(cuda),
                              dt.to(cuda), cu.to(cuda), state_dev, idx.to(cuda), initial_state_from_slot=from_slot)
    torch.cuda.synchronize()
    f = lambda t: t.double().numpy()
    ref_state = state.double().numpy()
    ref = gdn.gdn_prefill(f(q), f(k), f(v), f(a), f(b), f(A_log), f(dt), cu.numpy(), ref_state, idx.numpy(),
                          from_slot=from_slot)
    live = [i for i in range(8) if i in idx.tolist()]
    _prefill_close(out.float().cpu().numpy(), ref, state_dev.cpu().numpy()[live], ref_state[live])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gdn_prefill_chunk_edges(cuda, dtype):
    """Lengths on both sides of the 64-token chunk (one short of, equal to,
    one past, two chunks and the same +-1), state carried from the slots."""
    lens = [63, 64, 65, 127, 128, 129, 1]
    c = _prefill_inputs(lens, 2, 4, seed=16, slots=8, dtype=dtype)
    idx = torch.tensor([7, 0, 1, 2, 3, 4, 6], dtype=torch.int32)
    d = {k: v.to(cuda) for k, v in c.items()}
    state_dev = d["state"].clone()
    out = kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"], state_dev,
                              idx.to(cuda), initial_state_from_slot=True)
    torch.cuda.synchronize()
    f = lambda t: t.double().numpy()
    ref_state = c["state"].double().numpy()
    ref = gdn.gdn_prefill(f(c["q"]), f(c["k"]), f(c["v"]), f(c["a"]), f(c["b"]), f(c["A_log"]), f(c["dt"]),
                          c["cu"].numpy(), ref_state, idx.numpy(), from_slot=True)
    eo, es = _prefill_close(out.float().cpu().numpy(), ref, state_dev.cpu().numpy(), ref_state)
    if dtype == torch.float16:  # 11-bit operands: an order of magnitude closer
        assert eo <= 2e-3 and es <= 2e-3, (eo, es)
    assert torch.equal(state_dev[5].cpu(), c["state"][5])   # slot no sequence names


def test_gdn_prefill_then_decode_equals_longer_prefill(cuda):
    """Prefill of L tokens then one decode step == prefill of L + 1 tokens
    (same final state and last output, to the chunked form's precision)."""
    g = torch.Generator().manual_seed(7)
    L, H, HV, bf = 50, 1, 2, torch.bfloat16
    q, k = torch.randn(L + 1, H, 128, generator=g).to(bf), torch.randn(L + 1, H, 128, generator=g).to(bf)
    v = torch.randn(L + 1, HV, 128, generator=g).to(bf)
    a, b = torch.randn(L + 1, HV, generator=g).to(bf), torch.randn(L + 1, HV, generator=g).to(bf)
    A_log, dt = (torch.randn(HV, generator=g) * 0.5).to(cuda), (torch.randn(HV, generator=g) * 0.5).to(cuda)
    q, k, v, a, b = (x.to(cuda) for x in (q, k, v, a, b))
    st1 = torch.zeros(1, HV, 128, 128, device=cuda)
    st2 = torch.zeros(1, HV, 128, 128, device=cuda)
    idx = torch.zeros(1, dtype=torch.int32, device=cuda)
    kernels.gdn_prefill(q[:L], k[:L], v[:L], a[:L], b[:L], A_log, dt,
                        torch.tensor([0, L], dtype=torch.int32, device=cuda), st1, idx)
    o_dec = kernels.gdn_decode(q[L:], k[L:], v[L:], a[L:], b[L:], A_log, dt, st1, idx)
    o_all = kernels.gdn_prefill(q, k, v, a, b, A_log, dt,
                                torch.tensor([0, L + 1], dtype=torch.int32, device=cuda), st2, idx)
    torch.cuda.synchronize()
    sm = float(st2.abs().max())
    assert float((st1 - st2).abs().max()) <= 2e-2 * sm
    om = float(o_all.float().abs().max())
    assert float((o_dec[0].float() - o_all[L].float()).abs().max()) <= 2e-2 * om


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 128), (torch.bfloat16, 256),
                                     (torch.bfloat16, 64)])
def test_gated_rmsnorm_matches_oracle(cuda, dtype, d):
    """Against the oracle (same sum order, every operation rounded on its
    own): within one ulp on at most 0.5% of elements -- the last float32 bit
    of exp() in the silu is free; in place on the GDN output layout [T, HV, D]."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(37, 4, d, generator=g).to(dtype)
    z = (torch.randn(37, 4, d, generator=g) * 2).to(dtype)
    w = 0.5 + torch.rand(d, generator=g)
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    ref = gdn.gated_rmsnorm(x.float().numpy(), z.float().numpy(), w.numpy(), 1e-6, name)
    xd = x.to(cuda)
    out = kernels.gated_rmsnorm(xd, z.to(cuda), w.to(cuda), 1e-6, out=xd)
    torch.cuda.synchronize()
    assert out.data_ptr() == xd.data_ptr()
    it = torch.int16
    key = lambda t: (lambda b: torch.where(b < 0, -(b + 32768), b))(t.contiguous().view(it).int())
    ulps = (key(out.cpu()) - key(torch.from_numpy(ref).to(dtype))).abs()
    assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) <= 5e-3


@pytest.mark.parametrize("C,K,bf", [(1000, 4, torch.bfloat16), (1004, 4, torch.bfloat16), (2048, 3, torch.float16),
                                    (4096, 2, torch.bfloat16), (512, 8, torch.bfloat16)])
def test_conv1d_decode_and_prefill(cuda, C, K, bf):
    """Prefill of packed sequences from zero state, then decode steps on the
    pooled state: outputs within one ulp of the oracle on <= 0.5% of elements
    (exp's last bit is free), states bit-exact; prefill(L) then decode equals
    prefill(L + 1)'s last output.  Channel counts that are multiples of 8
    take the 8-channels-per-lane prefill kernel (runs of 16 tokens: the
    lengths cover a run's edges), 1004 the channel-pair one."""
    g = torch.Generator().manual_seed(9)
    lens = [1, 2, 7, 130, 16, 17, 33]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T = int(cu[-1])
    x = (torch.randn(T, C, generator=g) * 2).to(bf)
    w = (torch.randn(C, 1, K, generator=g) * 0.5).to(bf)
    state = torch.zeros(9, C, K - 1, dtype=bf)
    idx = torch.tensor([4, 0, -1, 2, 7, 8, 5], dtype=torch.int32)
    st_dev = state.clone().to(cuda)
    out = kernels.gdn_conv1d(x.to(cuda), w.to(cuda), st_dev, idx.to(cuda), cu_seqlens=cu.to(cuda))
    torch.cuda.synchronize()
    ref_state = state.float().numpy()
    dt = "bf16" if bf == torch.bfloat16 else "f16"
    ref = gdn.conv1d_silu(x.float().numpy(), w.reshape(C, K).float().numpy(), ref_state, idx.numpy(), cu.numpy(),
                          dtype=dt)
    key = lambda t: (lambda b: torch.where(b < 0, -(b + 32768), b))(t.contiguous().view(torch.int16).int())
    ulps = (key(out.cpu()) - key(torch.from_numpy(ref).to(bf))).abs()
    assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) <= 5e-3
    assert torch.equal(st_dev.cpu().float(), torch.from_numpy(ref_state))
    # decode: one new token for each sequence
    xd = (torch.randn(len(lens), C, generator=g) * 2).to(bf)
    od = kernels.gdn_conv1d(xd.to(cuda), w.to(cuda), st_dev, idx.to(cuda))
    torch.cuda.synchronize()
    refd = gdn.conv1d_silu(xd.float().numpy(), w.reshape(C, K).float().numpy(), ref_state, idx.numpy(), dtype=dt)
    live = idx >= 0
    ulps = (key(od.cpu()[live]) - key(torch.from_numpy(refd).to(bf)[live])).abs()
    assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) <= 5e-3
    assert torch.equal(st_dev.cpu().float(), torch.from_numpy(ref_state))


def test_gdn_core_layer_path(cuda):
    """layers.gdn_core (conv1d -> delta rule -> gated norm on the pools, with a
    module carrying the reference GatedDeltaNet's parameters): a prefill of
    three packed sequences, then two decode steps, against the oracle chain."""
    from types import SimpleNamespace
    from nano_qwen_amd.layers import gdn_core
    g = torch.Generator().manual_seed(10)
    H, HV, D, K, bf = 2, 4, 128, 4, torch.bfloat16
    C = 2 * H * D + HV * D
    layer = SimpleNamespace(
        num_k_heads=H, num_v_heads=HV, head_k_dim=D, head_v_dim=D,
        conv1d=SimpleNamespace(weight=(torch.randn(C, 1, K, generator=g) * 0.4).to(bf).to(cuda)),
        A_log=(torch.randn(HV, generator=g) * 0.5).to(cuda), dt_bias=(torch.randn(HV, generator=g) * 0.5).to(bf).to(cuda),
        norm=SimpleNamespace(weight=(0.5 + torch.rand(D, generator=g)).to(cuda), eps=1e-6),
        conv_states=torch.zeros(5, C, K - 1, dtype=bf, device=cuda),
        recurrent_states=torch.zeros(5, HV, D, D, device=cuda))
    lens = [3, 40, 17]
    idx = torch.tensor([4, 1, 2], dtype=torch.int32)
    ref_conv = np.zeros((5, C, K - 1), np.float32)
    ref_rec = np.zeros((5, HV, D, D))
    w = layer.conv1d.weight.reshape(C, K).float().cpu().numpy()
    A, dt = layer.A_log.float().cpu().numpy(), layer.dt_bias.float().cpu().numpy()
    nw = layer.norm.weight.cpu().numpy()

    def run(T, cu):
        x = (torch.randn(T, C, generator=g) * 2).to(bf)
        z = torch.randn(T, HV * D, generator=g).to(bf)
        a = torch.randn(T, HV, generator=g).to(bf)
        b = torch.randn(T, HV, generator=g).to(bf)
        out = gdn_core(layer, x.to(cuda), z.to(cuda), a.to(cuda), b.to(cuda), idx.to(cuda),
                       None if cu is None else cu.to(cuda))
        torch.cuda.synchronize()
        mixed = gdn.conv1d_silu(x.float().numpy(), w, ref_conv, idx.numpy(), None if cu is None else cu.numpy())
        q = mixed[:, :H * D].reshape(T, H, D)
        k = mixed[:, H * D:2 * H * D].reshape(T, H, D)
        v = mixed[:, 2 * H * D:].reshape(T, HV, D)
        f = lambda t: t.double().numpy()
        if cu is None:
            y = gdn.gdn_decode(q, k, v, f(a), f(b), A, dt, ref_rec, idx.numpy())
        else:
            y = gdn.gdn_prefill(q, k, v, f(a), f(b), A, dt, cu.numpy(), ref_rec, idx.numpy())
        from oracle.qk_norm_rope import round_to
        yb = round_to(y.astype(np.float32), "bf16").reshape(-1, D)
        ref = gdn.gated_rmsnorm(yb, z.float().numpy().reshape(-1, D), nw, 1e-6, "bf16").reshape(T, HV * D)
        o = out.float().cpu().numpy()
        assert np.all(np.abs(o - ref) <= 2 ** -6 * np.abs(ref) + 2e-2 * np.abs(ref).max()), float(np.abs(o - ref).max())
        # the chunked prefill's 16-bit operands (see _prefill_close); decode steps are float32
        assert np.abs(layer.recurrent_states.cpu().double().numpy() - ref_rec).max() <= 2e-2 * max(1.0, np.abs(ref_rec).max())
        assert torch.equal(layer.conv_states.cpu().float(), torch.from_numpy(ref_conv))

    run(sum(lens), torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32))
    run(3, None)
    run(3, None)


def test_gdn_decode_bench_shape(cuda):
    """The bench's decode shape: B = 64 sequences, 16 key heads, 32 value
    heads, every sequence on its own slot of a 64-slot pool."""
    c = _case(B=64, H=16, HV=32, slots=64, seed=11)
    c["idx"] = torch.randperm(64, generator=torch.Generator().manual_seed(12)).to(torch.int32)
    state_dev = c["state"].clone().to(cuda)
    out = _run(c, cuda, state_dev)
    ref_state = c["state"].double().numpy()
    ref = _ref(c, ref_state)
    _check(c, out, ref, state_dev, ref_state, np.ones(64, bool))


def _prefill_inputs(lens, H, HV, seed, slots, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T, bf = int(cu[-1]), dtype
    return dict(q=torch.randn(T, H, 128, generator=g).to(bf), k=torch.randn(T, H, 128, generator=g).to(bf),
                v=torch.randn(T, HV, 128, generator=g).to(bf), a=torch.randn(T, HV, generator=g).to(bf),
                b=torch.randn(T, HV, generator=g).to(bf), A_log=torch.randn(HV, generator=g) * 0.5,
                dt=torch.randn(HV, generator=g) * 0.5, state=torch.randn(slots, HV, 128, 128, generator=g) * 0.05,
                cu=cu)


@pytest.mark.slow
def test_gdn_prefill_cfg3_lengths(cuda):
    """cfg3's 16 sequence lengths (19,041 tokens, 256 .. 2048 each) with the
    bench's 16 key / 32 value heads, against the float64 chunked form run on
    the device (pinned against the step recurrence on the CPU)."""
    from oracle.inputs import make_prefill_case
    lens = make_prefill_case("cfg3", seed=0, device="cpu", prefix_blocks=(0, 0), nseq=16, hq=8, hkv=8, d=128)["lq"]
    H, HV = 16, 32
    c = _prefill_inputs(lens, H, HV, seed=13, slots=20)
    idx = torch.randperm(20, generator=torch.Generator().manual_seed(14))[:16].to(torch.int32)
    print(f"[gdn] prefill cfg3 lengths: {sum(lens)} tokens, H={H} HV={HV}", flush=True)
    d = {k: v.to(cuda) for k, v in c.items()}
    state_dev = d["state"].clone()
    out = kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"], state_dev,
                              idx.to(cuda), initial_state_from_slot=True)
    ref_state = d["state"].double().clone()
    ref = gdn.gdn_prefill_chunked(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], c["cu"], ref_state,
                                  idx, from_slot=True)
    torch.cuda.synchronize()
    live = idx.tolist()
    eo, es = _prefill_close(out.double().cpu().numpy(), ref.cpu().numpy(), state_dev.double().cpu().numpy()[live],
                            ref_state.cpu().numpy()[live])
    print(f"[gdn] cfg3 lengths: max error {eo:.2e} (outputs), {es:.2e} (states) of the largest magnitude", flush=True)


def test_gdn_prefill_empty_sequences(cuda):
    """Zero-length sequences (in the middle and last, where cu_seqlens[n] is
    one past the last row) write no output and store their initial state."""
    lens = [0, 9, 0, 70, 0]
    c = _prefill_inputs(lens, 2, 4, seed=15, slots=6)
    idx = torch.tensor([5, 0, 1, 3, 4], dtype=torch.int32)
    for from_slot in (False, True):
        d = {k: v.to(cuda) for k, v in c.items()}
        state_dev = d["state"].clone()
        out = kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"],
                                  state_dev, idx.to(cuda), initial_state_from_slot=from_slot)
        torch.cuda.synchronize()
        f = lambda t: t.double().numpy()
        ref_state = c["state"].double().numpy()
        ref = gdn.gdn_prefill(f(c["q"]), f(c["k"]), f(c["v"]), f(c["a"]), f(c["b"]), f(c["A_log"]), f(c["dt"]),
                              c["cu"].numpy(), ref_state, idx.numpy(), from_slot=from_slot)
        live = [i for i in range(6) if i in idx.tolist()]
        _prefill_close(out.float().cpu().numpy(), ref, state_dev.cpu().numpy()[live], ref_state[live])
        for slot in (5, 1, 4):   # the empty sequences' slots
            want = c["state"][slot] if from_slot else torch.zeros(4, 128, 128)
            assert torch.equal(state_dev[slot].cpu(), want)


def test_gdn_prefill_rejects_out_over_inputs(cuda):
    """The output rows double as the kernel's gate scratch, so an out that
    shares memory with an input is refused before the launch."""
    c = _prefill_inputs([70, 5], 2, 4, seed=21, slots=4)
    d = {k: v.to(cuda) for k, v in c.items()}
    idx = torch.tensor([0, 1], dtype=torch.int32, device=cuda)
    with pytest.raises(RuntimeError, match="must not overlap value"):
        kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"], d["state"], idx,
                            out=d["v"])


@pytest.mark.parametrize("nseq", [63, 64, 65, 90])
def test_gdn_prefill_batch_orders(cuda, nseq):
    """Batches of up to 64 sequences run longest first (the kernel ranks them
    by length, ties by index), larger ones in index order: both sides of that
    bound, with equal lengths among the sequences, against the float64
    chunked form on the device."""
    rng = np.random.default_rng(nseq)
    lens = [int(x) for x in rng.integers(1, 140, nseq)]
    lens[3] = lens[7] = lens[11] = 129  # ties
    H, HV = 2, 4
    c = _prefill_inputs(lens, H, HV, seed=nseq, slots=nseq + 3)
    idx = torch.randperm(nseq + 3, generator=torch.Generator().manual_seed(nseq))[:nseq].to(torch.int32)
    print(f"[gdn] prefill {nseq} sequences, {sum(lens)} tokens", flush=True)
    d = {k: v.to(cuda) for k, v in c.items()}
    state_dev = d["state"].clone()
    out = kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"], state_dev,
                              idx.to(cuda), initial_state_from_slot=True)
    ref_state = d["state"].double().clone()
    ref = gdn.gdn_prefill_chunked(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], c["cu"], ref_state,
                                  idx, from_slot=True)
    torch.cuda.synchronize()
    live = idx.tolist()
    _prefill_close(out.double().cpu().numpy(), ref.cpu().numpy(), state_dev.double().cpu().numpy()[live],
                   ref_state.cpu().numpy()[live])


@pytest.mark.parametrize("seed", range(12))
def test_gdn_prefill_random_sweep(cuda, seed):
    """Random shapes against the float64 chunked form on the device: key heads
    1-16 with 1, 2 or 4 value heads each (the XCD-paired head order is taken
    when the value heads are a multiple of 8 per group, and not otherwise),
    1-6 sequences of 1-400 tokens (chunk multiples among them), zero or pooled
    initial states, bf16 or f16, and q, k, v as strided views of one fused
    projection row in half the cases."""
    rng = np.random.default_rng(1000 + seed)
    G = int(rng.choice([1, 2, 4]))
    H = int(rng.choice([1, 2, 4, 8, 16]))
    HV = H * G
    nseq = int(rng.integers(1, 7))
    lens = [int(x) for x in rng.integers(1, 401, nseq)]
    if nseq > 1:
        lens[0] = 64 * int(rng.integers(1, 5))
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    from_slot = bool(seed % 3)
    fused = seed % 4 >= 2
    c = _prefill_inputs(lens, H, HV, seed=2000 + seed, slots=nseq + 2, dtype=dtype)
    d = {k: v.to(cuda) for k, v in c.items()}
    if fused:  # q | k | v of one projection row, as the layer slices them
        T = int(c["cu"][-1])
        row = torch.empty(T, (2 * H + HV) * 128, dtype=dtype, device=cuda)
        q = row[:, :H * 128].view(T, H, 128)
        k = row[:, H * 128:2 * H * 128].view(T, H, 128)
        v = row[:, 2 * H * 128:].view(T, HV, 128)
        q.copy_(d["q"]), k.copy_(d["k"]), v.copy_(d["v"])
        d["q"], d["k"], d["v"] = q, k, v
    idx = torch.randperm(nseq + 2, generator=torch.Generator().manual_seed(seed))[:nseq].to(torch.int32)
    print(f"[gdn] sweep {seed}: H={H} HV={HV} lens={lens} {dtype} from_slot={from_slot} fused={fused}", flush=True)
    state_dev = d["state"].clone()
    out = kernels.gdn_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], d["cu"], state_dev,
                              idx.to(cuda), initial_state_from_slot=from_slot)
    ref_state = d["state"].double().clone()
    ref = gdn.gdn_prefill_chunked(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt"], c["cu"], ref_state,
                                  idx, from_slot=from_slot)
    torch.cuda.synchronize()
    live = idx.tolist()
    _prefill_close(out.double().cpu().numpy(), ref.cpu().numpy(), state_dev.double().cpu().numpy()[live],
                   ref_state.cpu().numpy()[live])
    untouched = [sl for sl in range(nseq + 2) if sl not in live]
    for sl in untouched:  # slots no sequence names keep their contents
        assert torch.equal(state_dev[sl], d["state"][sl])
