"""Helpers shared by the GPU parity tests: move a (sub)case to the CPU, run
the oracle on it, and compare with the tolerances of the path's contract."""
from __future__ import annotations

import numpy as np
import torch

from oracle import fp8, paged

# bf16/f16 attention vs the float64 oracle (target's stated contract)
TOL_BF16 = dict(max_abs=2e-2, mean_abs=2e-3)
# fp8-e4m3 KV vs the oracle over the dequantized cache (looser, stated)
TOL_FP8 = dict(max_abs=3e-2, mean_abs=3e-3)


def f64(t: torch.Tensor) -> np.ndarray:
    t = t.detach().to("cpu")
    if t.dtype == torch.float8_e4m3fn:
        return fp8.decode_e4m3fn(t.view(torch.uint8).numpy()).astype(np.float64)
    return t.to(torch.float64).numpy()


def assert_close(out, ref, max_abs, mean_abs, what=""):
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    err = np.abs(out - ref)
    mx, mn = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"
    return mx, mn


def subpool(k_cache, v_cache, block_tables, lengths, seq_ids):
    """Copy the blocks used by ``seq_ids`` to a compact CPU pool.

    Returns (k_sub, v_sub, table_sub, remap) where remap maps an original
    block id to its sub-pool index (dict).
    """
    bs = k_cache.shape[1]
    blocks, rows = [], []
    for s in seq_ids:
        n = (int(lengths[s]) + bs - 1) // bs
        row = block_tables[s, :n].to("cpu").tolist()
        rows.append(row)
        blocks.extend(row)
    uniq = sorted(set(blocks))
    remap = {b: i for i, b in enumerate(uniq)}
    idx = torch.tensor(uniq, dtype=torch.int64, device=k_cache.device)
    k_sub = k_cache.index_select(0, idx).to("cpu")
    v_sub = v_cache.index_select(0, idx).to("cpu")
    width = max(len(r) for r in rows)
    table = np.full((len(seq_ids), width), -1, dtype=np.int64)
    for i, r in enumerate(rows):
        table[i, :len(r)] = [remap[b] for b in r]
    return k_sub, v_sub, table, remap


def remap_slots(slots, bs, remap):
    out = []
    for s in slots:
        s = int(s)
        out.append(remap[s // bs] * bs + s % bs if s >= 0 else -1)
    return np.asarray(out, dtype=np.int64)


def oracle_store_into(k_sub, v_sub, k_new, v_new, slots, k_scale=None, v_scale=None):
    """Apply the oracle store to CPU sub-pools; returns float64 value pools."""
    fp8_cache = k_sub.dtype == torch.float8_e4m3fn
    if fp8_cache:
        kc = k_sub.view(torch.uint8).numpy().copy()
        vc = v_sub.view(torch.uint8).numpy().copy()
        kq = fp8.quantize(k_new.to("cpu").float().numpy(), k_scale.to("cpu").numpy())
        vq = fp8.quantize(v_new.to("cpu").float().numpy(), v_scale.to("cpu").numpy())
        paged.store_kvcache(kq, vq, kc, vc, slots)
        return fp8.decode_e4m3fn(kc).astype(np.float64), fp8.decode_e4m3fn(vc).astype(np.float64)
    kc, vc = f64(k_sub), f64(v_sub)
    paged.store_kvcache(f64(k_new), f64(v_new), kc, vc, slots)
    return kc, vc


def decode_reference(case, seq_ids):
    """Oracle output [len(seq_ids), Hq, D] for a GPU decode case, computed
    from the cache contents *before* the GPU store (so store + decode are
    checked end to end)."""
    k_sub, v_sub, table, remap = case["_pre_store"]
    ctx = case["context_lens"].to("cpu").numpy()[seq_ids]
    slots_all = case["slot_mapping"].to("cpu").numpy()
    slots = remap_slots(slots_all[seq_ids], case["block_size"], remap)
    idx = torch.tensor(seq_ids, dtype=torch.int64)
    k_new = case["k_new"].to("cpu")[idx]
    v_new = case["v_new"].to("cpu")[idx]
    kc, vc = oracle_store_into(k_sub, v_sub, k_new, v_new, slots, case.get("k_scale"), case.get("v_scale"))
    ks = None if case.get("k_scale") is None else case["k_scale"].to("cpu").numpy()
    vs = None if case.get("v_scale") is None else case["v_scale"].to("cpu").numpy()
    q = f64(case["q"].to("cpu")[idx])
    return paged.paged_decode(q, kc, vc, table, ctx, case["scale"], ks, vs)


def snapshot_decode(case, seq_ids):
    """Record the pre-store sub-pool of ``seq_ids`` in the case."""
    case["_pre_store"] = subpool(case["k_cache"], case["v_cache"], case["block_tables"],
                                 case["context_lens"].to("cpu"), seq_ids)


def snapshot_prefill(case, seq_ids):
    """Record the pre-store sub-pool of ``seq_ids`` (paged cases)."""
    if case["block_tables"] is not None:
        lk = torch.tensor(case["lk"])
        case["_pre_store"] = subpool(case["k_cache"], case["v_cache"], case["block_tables"], lk, seq_ids)


def prefill_reference(case, seq_ids, rows_per_seq=None, seed=0):
    """Oracle output for the query rows of ``seq_ids``.

    Returns (global_row_indices, ref [n_rows, Hq, D]).  ``rows_per_seq``
    spot-checks a random subset of each sequence's rows (always including
    its first and last row).
    """
    cq = case["cu_seqlens_q"].to("cpu").numpy()
    lq = [case["lq"][s] for s in seq_ids]
    lk = [case["lk"][s] for s in seq_ids]
    rng = np.random.default_rng(seed)
    sub_cq = np.concatenate([[0], np.cumsum(lq)])
    sub_ck = np.concatenate([[0], np.cumsum(lk)])
    glob_rows = np.concatenate([np.arange(cq[s], cq[s + 1]) for s in seq_ids])
    local_rows = []
    for i, s in enumerate(seq_ids):
        n = lq[i]
        if rows_per_seq is None or rows_per_seq >= n:
            pick = np.arange(n)
        else:
            pick = np.unique(np.concatenate([[0, n - 1], rng.choice(n, rows_per_seq, replace=False)]))
        local_rows.append(sub_cq[i] + pick)
    local_rows = np.concatenate(local_rows)
    q = f64(case["q"].to("cpu")[torch.from_numpy(glob_rows)])
    ks = None if case.get("k_scale") is None else case["k_scale"].to("cpu").numpy()
    vs = None if case.get("v_scale") is None else case["v_scale"].to("cpu").numpy()
    if case["block_tables"] is None:
        k = f64(case["k_new"].to("cpu")[torch.from_numpy(glob_rows)])
        v = f64(case["v_new"].to("cpu")[torch.from_numpy(glob_rows)])
        ref = paged.varlen_prefill(q, k, v, sub_cq, sub_ck, case["scale"], rows=local_rows)
    else:
        k_sub, v_sub, table, remap = case["_pre_store"]
        slots = remap_slots(case["slot_mapping"].to("cpu").numpy()[glob_rows], case["block_size"], remap)
        idx = torch.from_numpy(glob_rows)
        kc, vc = oracle_store_into(k_sub, v_sub, case["k_new"].to("cpu")[idx], case["v_new"].to("cpu")[idx],
                                   slots, case.get("k_scale"), case.get("v_scale"))
        ref = paged.varlen_prefill(q, kc, vc, sub_cq, sub_ck, case["scale"], block_tables=table,
                                   rows=local_rows, k_scale=ks, v_scale=vs)
    return glob_rows[local_rows], ref[local_rows]


def full_decode_check(case, out, tol):
    """Every output row of a decode case against ``oracle/sdpa_path`` run in
    float32 on the device over the cache after the (separately bit-checked)
    store.  sdpa_path is pinned against the float64 oracle on the CPU."""
    from oracle import sdpa_path
    o = out.squeeze(1) if out.dim() == 4 else out
    ref = sdpa_path.paged_decode(case["q"], case["k_cache"], case["v_cache"], case["block_tables"],
                                 case["context_lens"].cpu(), case["scale"], case.get("k_scale"), case.get("v_scale"))
    err = (o.float() - ref).abs()
    mx, mn = float(err.max()), float(err.mean())
    assert bool(torch.isfinite(o.float()).all()), f"{case['name']}: non-finite output"
    assert mx <= tol["max_abs"] and mn <= tol["mean_abs"], \
        f"{case['name']} all rows: max-abs {mx:.3e} (<= {tol['max_abs']}), mean-abs {mn:.3e} (<= {tol['mean_abs']})"
    return mx, mn


def full_prefill_check(case, out, tol):
    """Every output row of a prefill case against ``oracle/sdpa_path`` in
    float32 on the device (after the store, like full_decode_check)."""
    from oracle import sdpa_path
    if case["block_tables"] is None:
        k, v, ks, vs = case["k_new"], case["v_new"], None, None
    else:
        k, v, ks, vs = case["k_cache"], case["v_cache"], case.get("k_scale"), case.get("v_scale")
    ref = sdpa_path.varlen_prefill(case["q"], k, v, case["cu_seqlens_q"].cpu(), case["cu_seqlens_k"].cpu(),
                                   case["scale"], block_tables=case["block_tables"], k_scale=ks, v_scale=vs)
    err = (out.float() - ref).abs()
    mx, mn = float(err.max()), float(err.mean())
    assert bool(torch.isfinite(out.float()).all()), f"{case['name']}: non-finite output"
    assert mx <= tol["max_abs"] and mn <= tol["mean_abs"], \
        f"{case['name']} all rows: max-abs {mx:.3e} (<= {tol['max_abs']}), mean-abs {mn:.3e} (<= {tol['mean_abs']})"
    return mx, mn
