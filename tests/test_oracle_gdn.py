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
