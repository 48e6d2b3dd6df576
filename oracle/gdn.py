"""Gated DeltaNet recurrent step, restated in numpy float64.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the
HIP entry point ``nq_gdn_decode``.

What it restates: decode_gated_delta_rule (layers/gated_delta_net.py:85-122)
-- FlashInfer's gated_delta_rule_decode_pretranspose with in-kernel gating
and ``use_qk_l2norm=True``, a third-party library absent here and unpinned
(its bit-level rounding is not pinned; the restatement is the gated delta
rule in exact arithmetic) -- with the inputs the layer prepares
(layers/gated_delta_net.py:178-248): the gating of ``_forward_prefill``
(g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b), :197-198), the
q/k l2 norm of layers/fla/l2norm.py (x / sqrt(sum(x^2) + 1e-6)), the
default scale K^-1/2 (layers/fla/chunk.py:106-107), the key-head
repeat_interleave for GQA (:199-201), and the state pool slot read and
written around the call (:168-173, 250-262).  State layout [V, K] (K-last).
"""
from __future__ import annotations

import numpy as np


def softplus(x):
    """torch.nn.functional.softplus (beta 1, threshold 20)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def l2norm(x, eps=1e-6):
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def gdn_step(S, q, k, v, a, b, A_log, dt_bias):
    """One token of one value head: returns (o [V], S_new [V, K])."""
    K = S.shape[1]
    qn, kn = l2norm(q), l2norm(k)
    g = -np.exp(np.float64(A_log)) * softplus(np.float64(a) + np.float64(dt_bias))
    beta = 1.0 / (1.0 + np.exp(-np.float64(b)))
    S = np.exp(g) * np.asarray(S, dtype=np.float64)
    u = beta * (np.asarray(v, dtype=np.float64) - S @ kn)
    S = S + np.outer(u, kn)
    return S @ (qn * K ** -0.5), S


def gdn_decode(q, k, v, a, b, A_log, dt_bias, state, state_indices):
    """Batch decode step: q, k [B, H, K]; v [B, HV, V]; a, b [B, HV];
    state [slots, HV, V, K] (updated in place, float64 copy semantics);
    returns out [B, HV, V] (NaN rows for skipped sequences)."""
    B, H, _ = q.shape
    HV, V = v.shape[1], v.shape[2]
    out = np.full((B, HV, V), np.nan)
    for bi in range(B):
        slot = int(state_indices[bi])
        if slot < 0 or slot >= state.shape[0]:
            continue
        for hv in range(HV):
            h = hv // (HV // H)
            o, S = gdn_step(state[slot, hv], q[bi, h], k[bi, h], v[bi, hv], a[bi, hv], b[bi, hv],
                            A_log[hv], dt_bias[hv])
            out[bi, hv] = o
            state[slot, hv] = S
    return out


def gdn_prefill(q, k, v, a, b, A_log, dt_bias, cu_seqlens, state, state_indices, from_slot=False):
    """Packed sequences: q, k [T, H, K]; v [T, HV, V]; a, b [T, HV].  Each
    sequence's state starts at zero (or the slot's contents), runs gdn_step
    over its tokens in order, and is stored to its slot (chunk_gated_delta_rule
    with initial_state=None, then the pool write; the chunked form computes
    the same recurrence)."""
    T, H, _ = q.shape
    HV, V = v.shape[1], v.shape[2]
    out = np.zeros((T, HV, V))
    for n in range(len(cu_seqlens) - 1):
        t0, t1 = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
        slot = int(state_indices[n])
        has = 0 <= slot < state.shape[0]
        for hv in range(HV):
            h = hv // (HV // H)
            S = np.array(state[slot, hv], dtype=np.float64) if (from_slot and has) else np.zeros((V, q.shape[2]))
            for t in range(t0, t1):
                out[t, hv], S = gdn_step(S, q[t, h], k[t, h], v[t, hv], a[t, hv], b[t, hv], A_log[hv], dt_bias[hv])
            if has:
                state[slot, hv] = S
    return out


def gated_rmsnorm(x, gate, weight, eps, dtype):
    """RMSNormGated.forward (layers/layernorm.py:143-157), eager, over the last
    axis: n = rnd(x / sqrt(mean(x^2) + eps)); rnd(rnd(n * rnd(w)) * silu(g)),
    silu(g) = g / (1 + exp(-g)) in float32 operations, rnd = round to dtype.
    The float32 sum of squares uses qk_norm_rope.sum_squares's order (one
    valid order for the reference's mean)."""
    from .qk_norm_rope import round_to, sum_squares
    F32 = np.float32
    xf = np.asarray(x, dtype=F32)
    var = sum_squares(xf) * F32(1.0 / xf.shape[-1])
    r = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    n = round_to(xf * r, dtype)
    nw = round_to(n * round_to(np.asarray(weight, dtype=F32), dtype), dtype)
    g = np.asarray(gate, dtype=F32)
    with np.errstate(over="ignore"):
        silu = (g / (F32(1.0) + np.exp(-g).astype(F32))).astype(F32)
    return round_to(nw * silu, dtype)


def conv1d_silu(x, weight, conv_state, state_indices, cu_seqlens=None, dtype="bf16"):
    """Causal depthwise conv1d + silu (layers/gated_delta_net.py:178-180,
    207-213, 218-227).  x [rows, C], weight [C, K], conv_state [slots, C, K-1]
    (updated in place).  Per output: y = rnd(sum_j w[j] x[t-K+1+j]) (float32,
    j in order), out = rnd(y / (1 + exp(-y))).  Decode (no cu_seqlens): row b
    continues the slot's state; prefill: each sequence starts from zeros and
    its slot keeps its last K - 1 inputs."""
    from .qk_norm_rope import round_to
    F32 = np.float32
    x = np.asarray(x, dtype=F32)
    w = np.asarray(weight, dtype=F32)
    rows, C = x.shape
    K = w.shape[1]
    out = np.zeros((rows, C), dtype=F32)
    seqs = [(b, b + 1) for b in range(rows)] if cu_seqlens is None else \
        [(int(cu_seqlens[i]), int(cu_seqlens[i + 1])) for i in range(len(cu_seqlens) - 1)]
    for n, (t0, t1) in enumerate(seqs):
        slot = int(state_indices[n])
        has = 0 <= slot < conv_state.shape[0]
        hist = (np.asarray(conv_state[slot], dtype=F32) if (has and cu_seqlens is None)
                else np.zeros((C, K - 1), dtype=F32))
        seq = np.concatenate([hist, x[t0:t1].T], axis=1)  # [C, K-1 + L]
        for i in range(t1 - t0):
            win = seq[:, i:i + K]
            y = np.zeros(C, dtype=F32)
            for j in range(K):
                y = (y + (w[:, j] * win[:, j]).astype(F32)).astype(F32)
            y = round_to(y, dtype)
            with np.errstate(over="ignore"):
                s = (y / (F32(1.0) + np.exp(-y).astype(F32))).astype(F32)
            out[t0 + i] = round_to(s, dtype)
        if has:
            conv_state[slot] = seq[:, -(K - 1):]
    return out


def gdn_prefill_chunked(q, k, v, a, b, A_log, dt_bias, cu_seqlens, state, state_indices, from_slot=False,
                        chunk=64):
    """The same prefill through the chunked (WY) form of the gated delta rule
    that the reference's prefill kernel computes (layers/fla/chunk.py:23-72:
    chunk_local_cumsum, then chunk_fwd.py's fused k k^T + triangular solve +
    w/u recompute, chunk_delta_h.py's state pass over chunks, chunk_o.py's
    outputs), in float64 torch on the tensors' device, all heads at once.

    Per chunk of length C with local log-decay cumsum G (G_i = sum_{j<=i} g_j),
    unit keys k_i, beta_i and the state S0 entering the chunk ([V, K]):
      A[i, j] = beta_i exp(G_i - G_j) (k_i . k_j)        for j < i, else 0
      T = (I + A)^-1
      W = T (beta exp(G) k),  U = T (beta v)             (rows = tokens)
      D = U - W S0^T                                     (the delta-rule updates)
      o_i = scale exp(G_i) S0 q_i + scale sum_{j<=i} exp(G_i - G_j) (k_j . q_i) D_j
      S_C = exp(G_C) S0 + sum_j exp(G_C - G_j) D_j k_j^T
    which unrolls gdn_step over the chunk exactly (in exact arithmetic), so
    the two restatements pin each other.  Inputs and outputs as gdn_prefill
    (numpy arrays or torch tensors; ``state`` updated in place)."""
    import torch
    as_t = lambda x: x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x))
    was_np = not isinstance(q, torch.Tensor)
    dev = as_t(q).device
    f = lambda x: as_t(x).to(device=dev, dtype=torch.float64)
    q, k, v, a, b = f(q), f(k), f(v), f(a), f(b)
    A_log, dt_bias = f(A_log), f(dt_bias)
    st = as_t(state)
    T, H, K = q.shape
    HV, V = v.shape[1], v.shape[2]
    rep = HV // H
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    qn = l2(q).repeat_interleave(rep, dim=1) * K ** -0.5      # [T, HV, K]
    kn = l2(k).repeat_interleave(rep, dim=1)
    g = -torch.exp(A_log) * torch.nn.functional.softplus(a + dt_bias)   # [T, HV]
    beta = torch.sigmoid(b)
    out = torch.zeros(T, HV, V, dtype=torch.float64, device=dev)
    cu = [int(x) for x in (cu_seqlens.tolist() if hasattr(cu_seqlens, "tolist") else cu_seqlens)]
    idx = [int(x) for x in (state_indices.tolist() if hasattr(state_indices, "tolist") else state_indices)]
    for n in range(len(cu) - 1):
        t0, t1 = cu[n], cu[n + 1]
        slot = idx[n]
        has = 0 <= slot < st.shape[0]
        S = (as_t(st[slot]).to(dev, torch.float64).clone() if (from_slot and has)
             else torch.zeros(HV, V, K, dtype=torch.float64, device=dev))
        for c0 in range(t0, t1, chunk):
            c1 = min(c0 + chunk, t1)
            kc = kn[c0:c1].transpose(0, 1)                      # [HV, C, K]
            qc = qn[c0:c1].transpose(0, 1)
            vc = v[c0:c1].transpose(0, 1)                       # [HV, C, V]
            bc = beta[c0:c1].transpose(0, 1)                    # [HV, C]
            G = torch.cumsum(g[c0:c1].transpose(0, 1), dim=1)   # [HV, C]
            C = c1 - c0
            decay = torch.exp(G[:, :, None] - G[:, None, :])    # [HV, C, C], exp(G_i - G_j)
            strict = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev), -1)
            A = torch.where(strict, bc[:, :, None] * decay * (kc @ kc.transpose(1, 2)), 0.0)
            Tm = torch.linalg.inv(torch.eye(C, dtype=torch.float64, device=dev) + A)
            W = Tm @ (bc[:, :, None] * torch.exp(G)[:, :, None] * kc)
            U = Tm @ (bc[:, :, None] * vc)
            Dl = U - W @ S.transpose(1, 2)                      # [HV, C, V]
            causal = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev))
            P = torch.where(causal, decay * (qc @ kc.transpose(1, 2)), 0.0)
            o = torch.exp(G)[:, :, None] * (qc @ S.transpose(1, 2)) + P @ Dl
            out[c0:c1] = o.transpose(0, 1)
            GC = G[:, -1]
            S = torch.exp(GC)[:, None, None] * S + (Dl * torch.exp(GC[:, None] - G)[:, :, None]).transpose(1, 2) @ kc
        if has:
            if isinstance(st, torch.Tensor) and not was_np:
                st[slot] = S.to(st.dtype)
            else:
                state[slot] = S.cpu().numpy()
    return out.cpu().numpy() if was_np else out
