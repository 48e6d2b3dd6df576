"""Pins of oracle/gdn.py (CPU).  The reference holds no test or fixture for
the delta rule, and FlashInfer (its decode kernel) is absent, so the
restatement is pinned by what the gated delta rule fixes algebraically."""
import numpy as np
import torch

from oracle import gdn

rng = np.random.default_rng(0)


def _vecs(K=128, V=128):
    S = rng.standard_normal((V, K)) * 0.1
    return S, rng.standard_normal(K), rng.standard_normal(K), rng.standard_normal(V)


def test_softplus_matches_torch():
    x = np.concatenate([rng.standard_normal(1000) * 10, [-100.0, 19.99, 20.0, 20.01, 100.0]])
    np.testing.assert_allclose(gdn.softplus(x), torch.nn.functional.softplus(torch.from_numpy(x)).numpy(),
                               rtol=1e-12, atol=1e-300)


def test_delta_rule_writes_the_value():
    """beta = 1, no decay: after the step, reading S with the same (normalized)
    key returns v -- the defining property of the delta rule (and of the S k
    vs k S orientation: a transposed state fails it)."""
    S, q, k, v = _vecs()
    o, S2 = gdn.gdn_step(S, q, k, v, a=0.0, b=60.0, A_log=-80.0, dt_bias=0.0)
    kn = gdn.l2norm(k)
    np.testing.assert_allclose(S2 @ kn, v, atol=1e-6 * np.abs(v - S @ kn).max() + 1e-12)


def test_zero_state_closed_form_and_gate_zero():
    """Zero state, no decay, beta = 1: o = v (k.q) K^-1/2 with unit q, k.
    beta = 0: the state only decays, S' = exp(g) S, and o = exp(g) S q K^-1/2."""
    S, q, k, v = _vecs()
    o, _ = gdn.gdn_step(np.zeros_like(S), q, k, v, a=0.0, b=60.0, A_log=-80.0, dt_bias=0.0)
    qn, kn = gdn.l2norm(q), gdn.l2norm(k)
    np.testing.assert_allclose(o, v * (kn @ qn) / np.sqrt(128), rtol=1e-9)
    a, A_log, dt = 0.7, 0.3, -0.2
    g = -np.exp(A_log) * np.log1p(np.exp(a + dt))
    o2, S2 = gdn.gdn_step(S, q, k, v, a=a, b=-60.0, A_log=A_log, dt_bias=dt)
    np.testing.assert_allclose(S2, np.exp(g) * S, rtol=1e-12)
    np.testing.assert_allclose(o2, np.exp(g) * S @ qn / np.sqrt(128), rtol=1e-12)


def test_decay_composes_and_gqa_map():
    """Two beta = 0 steps decay by exp(g1 + g2); value head hv reads key head
    hv // (HV / H) (the reference's repeat_interleave)."""
    S, q, k, v = _vecs()
    _, S1 = gdn.gdn_step(S, q, k, v, a=0.1, b=-60.0, A_log=0.2, dt_bias=0.0)
    _, S2 = gdn.gdn_step(S1, q, k, v, a=-0.4, b=-60.0, A_log=0.2, dt_bias=0.0)
    g1 = -np.exp(0.2) * np.log1p(np.exp(0.1))
    g2 = -np.exp(0.2) * np.log1p(np.exp(-0.4))
    np.testing.assert_allclose(S2, np.exp(g1 + g2) * S, rtol=1e-12)
    B, H, HV = 2, 2, 4
    q = rng.standard_normal((B, H, 128)); k = rng.standard_normal((B, H, 128))
    v = rng.standard_normal((B, HV, 128)); a = rng.standard_normal((B, HV)); b = rng.standard_normal((B, HV))
    A_log, dt = rng.standard_normal(HV) * 0.1, rng.standard_normal(HV) * 0.1
    pool = rng.standard_normal((3, HV, 128, 128)) * 0.1
    ref_pool = pool.copy()
    out = gdn.gdn_decode(q, k, v, a, b, A_log, dt, pool, np.array([2, -1]))
    o, S = gdn.gdn_step(ref_pool[2, 3], q[0, 1], k[0, 1], v[0, 3], a[0, 3], b[0, 3], A_log[3], dt[3])
    np.testing.assert_allclose(out[0, 3], o)
    np.testing.assert_allclose(pool[2, 3], S)
    assert np.isnan(out[1]).all() and np.array_equal(pool[:2], ref_pool[:2])


def test_gated_rmsnorm_oracle():
    """Against the reference's formula as eager torch CPU ops on bf16 tensors
    (≤ 1 ulp, almost always exact: the sum order and rsqrt are free); gate 0
    gives 0; weight 0 gives 0; scaling x by 2^k with eps = 0 changes nothing."""
    from oracle.qk_norm_rope import round_to
    F32 = np.float32
    x = round_to(rng.standard_normal((300, 128)).astype(F32), "bf16")
    z = round_to(rng.standard_normal((300, 128)).astype(F32) * 2, "bf16")
    w = (0.5 + rng.random(128)).astype(F32)
    got = gdn.gated_rmsnorm(x, z, w, 1e-6, "bf16")
    xt, zt = torch.from_numpy(x).bfloat16(), torch.from_numpy(z).bfloat16()
    xf = xt.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * torch.from_numpy(w).to(torch.bfloat16)
    ref = (ref * torch.nn.functional.silu(zt.float())).to(torch.bfloat16).float().numpy()
    gu = (got.view(np.uint32) >> 16).astype(np.int64)
    ru = (ref.view(np.uint32) >> 16).astype(np.int64)
    key = lambda u: np.where(u & 0x8000, 0x8000 - u, u)
    ulps = np.abs(key(gu) - key(ru))
    assert ulps.max() <= 1 and (ulps > 0).mean() < 5e-3
    assert np.all(gdn.gated_rmsnorm(x, np.zeros_like(z), w, 1e-6, "bf16") == 0)
    assert np.all(gdn.gated_rmsnorm(x, z, np.zeros_like(w), 1e-6, "bf16") == 0)
    y0 = gdn.gated_rmsnorm(x, z, w, 0.0, "bf16")
    assert np.array_equal(gdn.gated_rmsnorm(x * F32(8), z, w, 0.0, "bf16"), y0)


def test_chunked_form_equals_recurrence():
    """gdn_prefill (a loop over gdn_step) against gdn_prefill_chunked (the WY
    form the reference's chunk kernel computes: triangular solve per chunk,
    state carried across chunks) -- two independent restatements, equal to
    float64 round-off for chunk sizes 1, 16 and 64, lengths that cross chunk
    boundaries, zero or pooled initial states and a skipped slot."""
    lens = [1, 5, 64, 65, 130, 3, 0]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, H, HV = int(cu[-1]), 2, 4
    q, k = rng.standard_normal((T, H, 128)), rng.standard_normal((T, H, 128))
    v = rng.standard_normal((T, HV, 128))
    a, b = rng.standard_normal((T, HV)), rng.standard_normal((T, HV)) * 2
    A_log, dt = rng.standard_normal(HV) * 0.5, rng.standard_normal(HV) * 0.5
    st0 = rng.standard_normal((9, HV, 128, 128)) * 0.05
    idx = np.array([6, 0, -1, 3, 5, 7, 8])
    for from_slot in (False, True):
        s1 = st0.copy()
        o1 = gdn.gdn_prefill(q, k, v, a, b, A_log, dt, cu, s1, idx, from_slot=from_slot)
        for chunk in (1, 16, 64):
            s2 = st0.copy()
            o2 = gdn.gdn_prefill_chunked(q, k, v, a, b, A_log, dt, cu, s2, idx, from_slot=from_slot, chunk=chunk)
            assert np.abs(o1 - o2).max() <= 1e-12 * np.abs(o1).max()
            assert np.abs(s1 - s2).max() <= 1e-12 * np.abs(s1).max()
        # the empty last sequence keeps its initial state
        assert np.array_equal(s1[8], st0[8] if from_slot else np.zeros_like(st0[8]))
    # a dropped decay factor in the chunked form's state pass would fail here
    s3 = st0.copy()
    o3 = gdn.gdn_prefill_chunked(q, k, v, a, b, A_log - 50.0, dt, cu, s3, idx)   # g -> 0: pure delta rule
    s4 = st0.copy()
    o4 = gdn.gdn_prefill(q, k, v, a, b, A_log - 50.0, dt, cu, s4, idx)
    assert np.abs(o3 - o4).max() <= 1e-12 * np.abs(o4).max()
    assert np.abs(o3 - o1).max() > 1e-3 * np.abs(o1).max()


def _bits(x):
    """Signed-magnitude order key of bf16 values given as float32."""
    u = (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.int64)
    return np.where(u & 0x8000, 0x8000 - u, u)


def test_conv1d_silu_matches_torch_conv1d():
    """conv1d_silu against the reference's own torch ops on bf16 CPU tensors:
    prefill = F.silu(conv1d(x, padding=K-1, groups=C)[..., :S]) from zeros
    (layers/gated_delta_net.py:178-180), decode = F.silu(F.conv1d(cat(state,
    x), padding=0, groups=C)) on the last position with the state shifted
    (:218-227), and the prefill state = the last K-1 raw inputs (:207-213).
    Within one bf16 ulp (torch's accumulation order and exp are free), and
    bit-exact on integer-valued inputs, where every sum is exact."""
    from oracle.qk_norm_rope import round_to
    import torch.nn.functional as F
    C, K, L = 96, 4, 23
    x = round_to(rng.standard_normal((L, C)).astype(np.float32) * 2, "bf16")
    w = round_to(rng.standard_normal((C, K)).astype(np.float32) * 0.5, "bf16")
    st = np.zeros((3, C, K - 1), np.float32)
    got = gdn.conv1d_silu(x, w, st, np.array([1]), np.array([0, L]))
    xt = torch.from_numpy(x).bfloat16().T[None]                      # (1, C, S)
    wt = torch.from_numpy(w).bfloat16()[:, None, :]                  # (C, 1, K)
    ref = F.silu(F.conv1d(xt, wt, padding=K - 1, groups=C)[:, :, :L])[0].T.float().numpy()
    d = np.abs(_bits(got) - _bits(ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.02
    assert np.array_equal(st[1], x[-(K - 1):].T) and not st[0].any() and not st[2].any()
    # decode: one token per sequence on the pooled state
    xd = round_to(rng.standard_normal((1, C)).astype(np.float32) * 2, "bf16")
    prev = st[1].copy()
    gotd = gdn.conv1d_silu(xd, w, st, np.array([1]))
    win = torch.cat([torch.from_numpy(prev).bfloat16()[None], torch.from_numpy(xd).bfloat16().T[None]], dim=-1)
    refd = F.silu(F.conv1d(win, wt, padding=0, groups=C))[:, :, -1:][0].T.float().numpy()
    d = np.abs(_bits(gotd) - _bits(refd))
    assert d.max() <= 1 and (d > 0).mean() < 0.05
    assert np.array_equal(st[1], win[0, :, -(K - 1):].float().numpy())
    # integer-valued inputs: every product and sum is exact in float32 and
    # the pre-activation fits bf16, so the conv itself agrees bit for bit
    xi = rng.integers(-3, 4, (L, C)).astype(np.float32)
    wi = rng.integers(-2, 3, (C, K)).astype(np.float32)
    st = np.zeros((2, C, K - 1), np.float32)
    yi = gdn.conv1d_silu(xi, wi, st, np.array([0]), np.array([0, L]))
    pre = F.conv1d(torch.from_numpy(xi).double().T[None], torch.from_numpy(wi).double()[:, None, :],
                   padding=K - 1, groups=C)[:, :, :L][0].T
    exact = F.silu(pre.bfloat16().float()).bfloat16().float().numpy()
    d = np.abs(_bits(yi) - _bits(exact))
    assert d.max() <= 1 and (d > 0).mean() < 0.02
    # a window off by one tap (a plausible indexing mistake) is far off
    shifted = np.concatenate([np.zeros((1, C), np.float32), xi[:-1]])
    ys = gdn.conv1d_silu(shifted, wi, np.zeros((2, C, K - 1), np.float32), np.array([0]), np.array([0, L]))
    assert (np.abs(_bits(ys) - _bits(exact)) > 1).mean() > 0.5
