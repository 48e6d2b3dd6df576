"""Pins of oracle/qk_norm_rope.py (CPU): each check is one that a plausible
mistake in the restatement (a dropped rounding, the weight used without its
+1 offset, the wrong rotation sign or half, sum instead of mean) would fail.

The reference holds no test or fixture for GemmaRMSNorm or the rotary
embedding, so the oracle is pinned by library routines, closed forms and
invariants only.
"""
import numpy as np
import pytest
import torch

from oracle import fp8
from oracle import qk_norm_rope as o

F32 = np.float32


def _bf16_ulps(a, b):
    """|a - b| in bf16 units in the last place (a, b float32 holding bf16 values)."""
    def key(x):
        u = (x.view(np.uint32) >> 16).astype(np.int64)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(key(np.ascontiguousarray(a, F32)) - key(np.ascontiguousarray(b, F32)))


def test_round_to_bf16_matches_torch_cast():
    """Nearest-even rounding to bf16 against torch's cast (a library routine),
    including ties, subnormals, infinities, NaN and the largest finite values."""
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200_000) * 10).astype(F32),
        rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(F32),
        np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 1e-40, -1e-40, np.inf, -np.inf,
                  3.4028235e38, -3.4028235e38, 0.0, -0.0], dtype=F32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = o.round_to(x, "bf16")
    fin = ~np.isnan(x)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.isnan(got[~fin]).all()
    assert np.array_equal(o.round_to(x[fin], "f16"), torch.from_numpy(x[fin]).half().float().numpy())


def test_rope_cache_matches_closed_form():
    """cos_sin_cache[p] = [cos(p f_j), sin(p f_j)] with f_j = base^(-2j/R), up to
    the float32 rounding of f_j and of p * f_j."""
    R, base, P = 64, 1e7, 8192
    cs = o.rope_cache(R, P, base).astype(np.float64)
    p = np.arange(P, dtype=np.float64)[:, None]
    f = base ** (-np.arange(0, R, 2, dtype=np.float64) / R)[None, :]
    ang = p * f
    bound = 4e-7 * np.abs(ang) + 1e-6     # float32 inv_freq and product roundings
    assert np.all(np.abs(cs[:, :R // 2] - np.cos(ang)) <= bound)
    assert np.all(np.abs(cs[:, R // 2:] - np.sin(ang)) <= bound)
    assert np.all(cs[0, :R // 2] == 1.0) and np.all(cs[0, R // 2:] == 0.0)


def test_norm_is_rms_scaling():
    """fp32, eps = 0, w = 0: y = x / rms(x) (mean of squares, not sum), against
    the float64 closed form x * sqrt(D) / ||x||."""
    rng = np.random.default_rng(1)
    for d in (64, 128, 256):
        x = rng.standard_normal((50, 4, d)).astype(F32) * F32(3)
        y = o.gemma_rms_norm(x, np.zeros(d, F32), 0.0, "f32")
        ref = x.astype(np.float64) * np.sqrt(d) / np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
        np.testing.assert_allclose(y, ref, rtol=3e-6, atol=1e-6)


def test_norm_weight_offset_and_eps():
    """Gemma semantics: the factor is (1 + w).  w = -1 zeroes the row, w = 1
    doubles it exactly; eps enters under the square root."""
    rng = np.random.default_rng(2)
    x = o.round_to(rng.standard_normal((20, 3, 128)).astype(F32), "bf16")
    base = o.gemma_rms_norm(x, np.zeros(128, F32), 1e-6, "bf16")
    assert np.all(o.gemma_rms_norm(x, -np.ones(128, F32), 1e-6, "bf16") == 0)
    assert np.array_equal(o.gemma_rms_norm(x, np.ones(128, F32), 1e-6, "bf16"), 2 * base)
    # weight_offset = 0 is the plain RMSNorm: w = 1 then gives the same row as Gemma w = 0
    assert np.array_equal(o.gemma_rms_norm(x, np.ones(128, F32), 1e-6, "bf16", weight_offset=0.0), base)
    # a row of zeros: y = 0 * 1/sqrt(eps) = 0; a constant row c: y = c / sqrt(c^2 + eps)
    z = o.gemma_rms_norm(np.zeros((1, 128), F32), np.zeros(128, F32), 1e-6, "f32")
    assert np.all(z == 0)
    c = o.gemma_rms_norm(np.full((1, 128), 1e-3, F32), np.zeros(128, F32), 1e-6, "f32")
    np.testing.assert_allclose(c, 1e-3 / np.sqrt(1e-6 + 1e-6), rtol=1e-6)


def test_norm_scale_invariance_bit_exact():
    """eps = 0: scaling a row by 2^k changes nothing, bit for bit (every float32
    step scales exactly)."""
    rng = np.random.default_rng(3)
    x = o.round_to(rng.standard_normal((30, 8, 128)).astype(F32), "bf16")
    w = o.round_to(rng.uniform(-1, 1, 128).astype(F32), "bf16")
    y = o.gemma_rms_norm(x, w, 0.0, "bf16")
    for k in (-6, -1, 3, 10):
        assert np.array_equal(o.gemma_rms_norm(x * F32(2.0 ** k), w, 0.0, "bf16"), y)


def test_norm_rounding_points_match_torch_ops():
    """With weights for which 1 + w is exact in bf16 (eager and compiled
    semantics then coincide), the oracle matches the reference's formula run
    as eager torch CPU ops to within one bf16 ulp, almost always exactly; the
    residue is the float32 sum order and rsqrt.  Dropping the rounding of
    x.to(dtype) would disagree on a large fraction of elements."""
    rng = np.random.default_rng(4)
    x = o.round_to(rng.standard_normal((400, 8, 128)).astype(F32) * F32(2), "bf16")
    w = (rng.integers(-127, 128, 128) / 128.0).astype(F32)      # 1 + w exact in bf16
    got = o.gemma_rms_norm(x, w, 1e-6, "bf16")
    xt = torch.from_numpy(x).to(torch.bfloat16)
    wt = torch.from_numpy(w).to(torch.bfloat16)
    xf = xt.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    ref = ((xf * torch.rsqrt(var + 1e-6)).to(torch.bfloat16) * (1.0 + wt)).float().numpy()
    ulps = _bf16_ulps(got, ref)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 5e-3
    no_round = o.round_to((xf * torch.rsqrt(var + 1e-6)).numpy() * (1 + w), "bf16")
    assert (_bf16_ulps(no_round, ref) > 0).mean() > 0.05


def test_rope_is_complex_rotation():
    """The rotary part is z = (x1 + i x2) * exp(i theta), theta = p * f_j, as a
    complex128 product; dims >= R pass through unchanged."""
    rng = np.random.default_rng(5)
    N, H, D, R = 40, 3, 128, 32
    x = rng.standard_normal((N, H, D)).astype(F32)
    pos = rng.integers(0, 64, N)
    cs = o.rope_cache(R, 64, 1e7)
    z = o.apply_partial_rope(x, cs[pos], R, "f32").astype(np.float64)
    f = 1e7 ** (-np.arange(0, R, 2, dtype=np.float64) / R)
    th = pos[:, None, None] * f[None, None, :]
    ref = (x[..., :R // 2] + 1j * x[..., R // 2:R].astype(np.float64)) * np.exp(1j * th)
    np.testing.assert_allclose(z[..., :R // 2], ref.real, atol=2e-5)
    np.testing.assert_allclose(z[..., R // 2:R], ref.imag, atol=2e-5)
    assert np.array_equal(z[..., R:], x[..., R:].astype(np.float64))


def test_rope_position_zero_identity_and_pair_norms():
    rng = np.random.default_rng(6)
    x = o.round_to(rng.standard_normal((16, 4, 256)).astype(F32), "bf16")
    cs = o.rope_cache(64, 4096, 1e7)
    assert np.array_equal(o.apply_partial_rope(x, cs[np.zeros(16, int)], 64, "bf16"), x)
    pos = rng.integers(0, 4096, 16)
    z = o.apply_partial_rope(x, cs[pos], 64, "f32")
    n_in = x[..., :32] ** 2 + x[..., 32:64] ** 2
    n_out = z[..., :32] ** 2 + z[..., 32:64] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)


def test_qk_norm_rope_composition_and_bad_positions():
    """qk_norm_rope = norm then rope with each token's row; rows with a
    position outside the table are NaN; R = 0 is the norm alone."""
    rng = np.random.default_rng(7)
    N, D, R = 12, 128, 32
    q = o.round_to(rng.standard_normal((N, 4, D)).astype(F32), "bf16")
    k = o.round_to(rng.standard_normal((N, 2, D)).astype(F32), "bf16")
    qw = o.round_to(rng.uniform(-1, 1, D).astype(F32), "bf16")
    kw = o.round_to(rng.uniform(-1, 1, D).astype(F32), "bf16")
    cs = o.rope_cache(R, 100, 1e7)
    pos = rng.integers(0, 100, N)
    pos[3], pos[7] = -1, 100
    qo, ko = o.qk_norm_rope(q, k, pos, cs, R, qw, kw, 1e-6, "bf16")
    good = np.ones(N, bool)
    good[[3, 7]] = False
    assert np.isnan(qo[~good]).all() and np.isnan(ko[~good]).all()
    ref_q = o.apply_partial_rope(o.gemma_rms_norm(q, qw, 1e-6, "bf16"), cs[np.clip(pos, 0, 99)], R, "bf16")
    assert np.array_equal(qo[good], ref_q[good])
    q0, _ = o.qk_norm_rope(q, k, np.abs(pos), np.zeros((0, 0), F32), 0, qw, kw, 1e-6, "bf16")
    assert np.array_equal(q0, o.gemma_rms_norm(q, qw, 1e-6, "bf16"))


def test_store_rows_same_dtype_and_fp8():
    rng = np.random.default_rng(8)
    n, hkv, d = 10, 2, 64
    k = rng.standard_normal((n, hkv, d)).astype(F32)
    v = rng.standard_normal((n, hkv, d)).astype(F32)
    slots = rng.permutation(40)[:n].astype(np.int32)
    slots[2] = -1
    kc = np.zeros((40, hkv, d), F32)
    vc = np.zeros((40, hkv, d), F32)
    o.store_rows(k, v, kc, vc, slots)
    ok = slots >= 0
    assert np.array_equal(kc[slots[ok]], k[ok]) and np.array_equal(vc[slots[ok]], v[ok])
    assert np.count_nonzero(np.abs(kc).sum(axis=(1, 2))) == ok.sum()
    kq = np.zeros((40, hkv, d), np.uint8)
    vq = np.zeros((40, hkv, d), np.uint8)
    ks = fp8.absmax_scale(k)
    vs = fp8.absmax_scale(v)
    o.store_rows(k, v, kq, vq, slots, ks, vs)
    assert np.array_equal(kq[slots[ok]], fp8.quantize(k[ok], ks))
    assert np.array_equal(vq[slots[ok]], fp8.quantize(v[ok], vs))


def test_sum_squares_order_is_a_sum():
    """The fixed-order sum equals the exact sum within float32 accumulation
    error, every butterfly lane ends equal, and it is exact on integers."""
    rng = np.random.default_rng(9)
    for d in (64, 128, 256):
        x = rng.standard_normal((100, d)).astype(F32)
        s = o.sum_squares(x)[:, 0].astype(np.float64)
        ref = (x.astype(np.float64) ** 2).sum(-1)
        np.testing.assert_allclose(s, ref, rtol=d * 6e-8)
        xi = rng.integers(-50, 50, (10, d)).astype(F32)
        assert np.array_equal(o.sum_squares(xi)[:, 0], (xi.astype(np.int64) ** 2).sum(-1).astype(F32))


def test_output_gate_oracle():
    """sigmoid32 against the float64 logistic function (scipy's expit, a library
    routine) within float32 error; sigmoid(0) = 1/2 exactly; a gate of +30 is
    the identity in bf16, -200 (exp overflows) gives exact zeros, -30 scales by
    about 9.4e-14; and against the reference's eager torch ops on bf16 tensors."""
    from scipy.special import expit
    from oracle.output_gate import output_gate, sigmoid32
    rng = np.random.default_rng(10)
    g = (rng.standard_normal(100_000) * 6).astype(F32)
    np.testing.assert_allclose(sigmoid32(g), expit(g.astype(np.float64)), rtol=4e-7, atol=1e-30)
    assert sigmoid32(np.zeros(3, F32))[0] == 0.5
    ob = o.round_to(rng.standard_normal(1000).astype(F32), "bf16")
    assert np.array_equal(output_gate(ob, np.full(1000, 30, F32), "bf16"), ob)
    assert np.all(output_gate(ob, np.full(1000, -200, F32), "bf16") == 0)
    np.testing.assert_allclose(output_gate(ob, np.full(1000, -30, F32), "bf16"), ob * expit(-30.0), rtol=8e-3)
    assert np.array_equal(output_gate(ob, np.zeros(1000, F32), "bf16"), ob * F32(0.5))
    gb = o.round_to(g[:1000], "bf16")
    ref = torch.from_numpy(ob).to(torch.bfloat16) * torch.sigmoid(torch.from_numpy(gb).to(torch.bfloat16))
    u = _bf16_ulps(output_gate(ob, gb, "bf16"), ref.float().numpy())
    assert u.max() <= 1 and (u > 0).mean() < 5e-3
