"""Benchmark of the paged attention path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--no-cpu] [--only cfg2]

A "step" is one pass of the path over one batch of synthetic input:
  decode  (cfg2/cfg4/cfg5): store of the new token + paged decode, one launch
                            (nq_paged_decode_store, Attention.forward's decode path;
                            ``two_call_ms``: the store and the decode as two launches)
  prefill (cfg3):           store_kvcache of the new tokens + causal varlen prefill
Inputs are resident in HBM before timing starts.  Decode steps alternate
between two independent KV pools (each larger than the 256 MB MALL), so no
step re-reads KV the previous step left in the Infinity Cache; the same step
replayed as a HIP graph (the runner's path) is reported as ``graph_ms``: the
time per step in a graph of 4 steps, as the runner's whole-model graphs run
every layer's step per replay (``graph1_ms``: one step per graph, which also
carries the replay's own launch time).
Every measurement warms up for at least 20 ms
and times its steps back to back in five groups between events:
``ms_per_step`` is the mean over all timed steps (the whole-step rates, and
the headline, use it) and ``ms_median`` the median of the groups' means (the
per-kernel rates under ``extra`` use it).

The headline (``value``) is cfg2's algorithmic HBM bandwidth in GB/s; cfg3's
TFLOP/s and the other decode configurations are reported under ``extra``, as
is the fused q/k norm + rotary + KV store call over cfg3's and cfg2's new
tokens (``cfg3_norm_rope``, ``cfg2_norm_rope``: HBM GB/s), and Qwen3.5's output
gate (``cfg2_gate``: gated vs plain decode; ``cfg3_gate``: gated vs plain
prefill, and the stand-alone in-place gate pass for comparison), head_dim 256
(``cfg2_d256``, ``cfg5_d256``, ``cfg3_d256``) and the Gated DeltaNet decode
step (``gdn_decode``: HBM GB/s over the state pool) and prefill
(``gdn_prefill``: chunked form over cfg3's sequence lengths), and the gated
RMS norm of its output (``gdn_norm``) and the causal conv1d before it
(``gdn_conv``), HBM GB/s; cfg3 with an fp8 KV cache (``cfg3_fp8``); and the
prefill kernel on long sequences (``cfg3_long``: 4 x 8192 new tokens, half
with a prefix, causal), where item transitions are few.
``roofline`` covers the kernels of the headline workload (paged decode with
the fused store: main kernel + split-K merge, i.e. the whole step), timed
with HIP events on the stream the kernels run on.  ``cpu_baseline`` times the CPU restatement of the path
(torch gather + repeat_interleave + scaled_dot_product_attention) on the
host cores for a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
GRAPH_LAYERS = 4  # decode steps (layers) captured per graph for graph_ms
BF16_PEAK_TFLOPS = 2500.0


_LAST = {}  # the mean ms per step of the last _events_time call (timed region / steps)
MIN_WARM_MS = 20.0


def _events_time(fn, steps, warmup, groups=5):
    """Warm up for at least `warmup` steps and MIN_WARM_MS of them (so the
    clocks have ramped), then time `steps` steps back to back in `groups`
    consecutive groups, with an event on the current stream between groups
    (an event between every step would add its own gap to each step).
    Returns the median over the groups of their ms per step; _LAST["mean"]
    holds the mean (the whole timed region / steps).  fn(i) gets a running
    step index (pools alternate on it)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    i = warmup
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < MIN_WARM_MS:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    groups = max(1, min(groups, steps))
    bounds = [round(steps * g / groups) for g in range(groups + 1)]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    ev[0].record()
    for g in range(groups):
        for k in range(bounds[g], bounds[g + 1]):
            fn(i + k)
        ev[g + 1].record()
    torch.cuda.synchronize()
    per = [ev[g].elapsed_time(ev[g + 1]) / (bounds[g + 1] - bounds[g]) for g in range(groups)]
    _LAST["mean"] = ev[0].elapsed_time(ev[groups]) / steps
    return statistics.median(per)


def _second_pool(case):
    import torch
    k2 = torch.empty_like(case["k_cache"])
    v2 = torch.empty_like(case["v_cache"])
    k2.view(torch.uint8).copy_(case["k_cache"].view(torch.uint8).roll(1, 0))
    v2.view(torch.uint8).copy_(case["v_cache"].view(torch.uint8).roll(1, 0))
    return k2, v2


def bench_decode(name, steps, warmup, seed=0, **override):
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import decode_bytes, decode_flops, make_decode_case

    dev = torch.device("cuda:0")
    case = make_decode_case(name, seed=seed, device=dev, **override)
    pools = [(case["k_cache"], case["v_cache"]), _second_pool(case)]
    out = torch.empty(case["batch"], 1, case["hq"], case["d"], dtype=case["q"].dtype, device=dev)
    q = case["q"].unsqueeze(1)

    def step(i):
        # the runner's decode step: store of the new token + decode, one launch
        # (Attention.forward's decode path, nq_paged_decode_store)
        kc, vc = pools[i % 2]
        kernels.paged_decode(q, kc, vc, case["context_lens"], case["block_tables"], case["scale"],
                             case["k_scale"], case["v_scale"], out=out, k=case["k_new"], v=case["v_new"],
                             slot_mapping=case["slot_mapping"])

    def two_calls(i):
        kc, vc = pools[i % 2]
        kernels.store_kvcache(case["k_new"], case["v_new"], kc, vc, case["slot_mapping"], case["k_scale"],
                              case["v_scale"])
        kernels.paged_decode(q, kc, vc, case["context_lens"], case["block_tables"], case["scale"],
                             case["k_scale"], case["v_scale"], out=out)

    def attn_only(i):
        kc, vc = pools[i % 2]
        kernels.paged_decode(q, kc, vc, case["context_lens"], case["block_tables"], case["scale"],
                             case["k_scale"], case["v_scale"], out=out)

    ms = _events_time(step, steps, warmup)
    ms_mean = _LAST["mean"]
    # The step as graph replays (engine run_model's path).  The runner
    # captures the whole model per batch bucket, so each replay runs every
    # layer's attention step: graph_ms is the time per step in a graph of
    # GRAPH_LAYERS steps (alternating pools, as consecutive layers read
    # different caches); graph1_ms the same with one step per graph, which
    # also carries the replay's own launch time (a few microseconds of idle
    # GPU per replay on this ROCm).
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        step(0)  # the capture stream's workspace exists before the capture
    side.synchronize()
    multi = torch.cuda.CUDAGraph()
    with torch.cuda.graph(multi, stream=side):
        for layer in range(GRAPH_LAYERS):
            step(layer)
    graphs = []
    for p in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step(p)
        graphs.append(g)
    torch.cuda.synchronize()
    ms_graph = _events_time(lambda i: multi.replay(), max(1, steps // GRAPH_LAYERS), warmup) / GRAPH_LAYERS
    ms_graph1 = _events_time(lambda i: graphs[i % 2].replay(), steps, warmup)
    ms_attn = _events_time(attn_only, steps, warmup)
    ms_two = _events_time(two_calls, steps, warmup)
    nbytes = decode_bytes(case)
    store_bytes = 2 * case["batch"] * case["hkv"] * case["d"] * (case["q"].element_size() +
                                                                 case["k_cache"].element_size())
    attn_bytes = nbytes - store_bytes
    W = case["block_tables"].shape[1]
    ns, st = kernels.decode_plan(case["batch"], case["hq"], case["hkv"], W, case["block_size"],
                                 case["k_cache"].dtype)
    res = dict(
        ms_per_step=ms_mean, ms_median=ms, graph_ms=ms_graph, gbs=nbytes / (ms_mean * 1e-3) / 1e9,
        tokens_per_s=case["batch"] / (ms_mean * 1e-3), median_gbs=nbytes / (ms * 1e-3) / 1e9,
        hbm_frac=nbytes / (ms_mean * 1e-3) / 1e9 / HBM_PEAK_GBS, bytes_per_step=nbytes,
        graph_hbm_frac=nbytes / (ms_graph * 1e-3) / 1e9 / HBM_PEAK_GBS, graph_layers=GRAPH_LAYERS,
        graph1_ms=ms_graph1, graph1_hbm_frac=nbytes / (ms_graph1 * 1e-3) / 1e9 / HBM_PEAK_GBS,
        tflops=decode_flops(case) / (ms * 1e-3) / 1e12,
        step_median_gbs=nbytes / (ms * 1e-3) / 1e9,
        attn_ms=ms_attn, attn_gbs=attn_bytes / (ms_attn * 1e-3) / 1e9, attn_bytes=attn_bytes,
        two_call_ms=ms_two, two_call_hbm_frac=nbytes / (ms_two * 1e-3) / 1e9 / HBM_PEAK_GBS,
        splits=ns, split_tokens=st, batch=case["batch"], hq=case["hq"], hkv=case["hkv"],
        kv_dtype=str(case["k_cache"].dtype).replace("torch.", ""),
        sum_ctx=int(case["context_lens"].sum()))
    return res, case


def bench_prefill(name, steps, warmup, seed=0, **override):
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import make_prefill_case, prefill_bytes, prefill_flops

    dev = torch.device("cuda:0")
    case = make_prefill_case(name, seed=seed, device=dev, **override)
    out = torch.empty_like(case["q"])

    def attn(i):
        kernels.varlen_prefill(case["q"], case["k_cache"], case["v_cache"], case["cu_seqlens_q"],
                               case["cu_seqlens_k"], case["max_seqlen_q"], case["max_seqlen_k"], case["scale"],
                               causal=True, block_table=case["block_tables"], k_scale=case["k_scale"],
                               v_scale=case["v_scale"], out=out)

    def step(i):
        kernels.store_kvcache(case["k_new"], case["v_new"], case["k_cache"], case["v_cache"],
                              case["slot_mapping"], case["k_scale"], case["v_scale"])
        attn(i)

    ms = _events_time(step, steps, warmup)
    ms_mean = _LAST["mean"]
    ms_attn = _events_time(attn, steps, warmup)
    fl = prefill_flops(case)
    return dict(ms_per_step=ms_mean, ms_median=ms, tflops=fl / (ms_mean * 1e-3) / 1e12, attn_ms=ms_attn,
                attn_tflops=fl / (ms_attn * 1e-3) / 1e12, mfma_frac=fl / (ms_attn * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                flops=fl, tokens_per_s=sum(case["lq"]) / (ms_mean * 1e-3), total_q=sum(case["lq"]),
                gbs=prefill_bytes(case) / (ms_mean * 1e-3) / 1e9), case


def bench_norm_rope(name, steps, warmup, seed=0):
    """The fused q/k norm + rotary + KV store call over the new tokens of a
    configuration (Qwen3.5 partial rotary factor 0.25: R = 32 of D = 128).
    The timed loop calls the C ABI directly with the checked arguments."""
    import torch
    from nano_qwen_amd import kernels
    from nano_qwen_amd._lib import lib
    from oracle.inputs import make_norm_rope_case, norm_rope_bytes

    c = make_norm_rope_case(name, seed=seed, device="cuda")
    d = c["d"]
    q_out = torch.empty(c["n"], c["hq"], d, dtype=c["key"].dtype, device="cuda")
    k_out = torch.empty_like(c["key"])
    args = kernels.qk_norm_rope_store(
        c["positions"], c["q_gate"][..., :d], c["key"], c["value"], c["q_weight"], c["k_weight"], c["eps"],
        c["cos_sin_cache"], c["rotary_dim"], k_cache=c["k_cache"], v_cache=c["v_cache"],
        slot_mapping=c["slot_mapping"], k_scale=c["k_scale"], v_scale=c["v_scale"], q_out=q_out, k_out=k_out,
        _return_args=True)
    fn = lib().nq_qk_norm_rope_store

    def step(i):
        rc = fn(*args)
        if rc:
            raise RuntimeError(f"qk_norm_rope_store failed ({rc})")

    # A call lasts under 0.1 ms: warm up for about 20 ms so the clocks have
    # ramped before the timed steps.
    ms = _events_time(step, steps, max(warmup, 200))
    nb = norm_rope_bytes(c)
    return dict(ms_per_step=ms, gbs=nb / (ms * 1e-3) / 1e9, hbm_frac=nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                bytes=nb, tokens=c["n"], rotary_dim=c["rotary_dim"],
                tokens_per_s=c["n"] / (ms * 1e-3)), c


def bench_gate(name, steps, warmup, seed=0):
    """Qwen3.5's output gate: for decode (cfg2) the gated decode step against
    the plain one (the gate rides in the kernel's store); for prefill (cfg3)
    the in-place gate pass over the whole output [sum Lq, Hq, D]."""
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import make_decode_case, make_prefill_case

    g = torch.Generator(device="cuda").manual_seed(seed + 9)
    if name == "cfg2":
        c = make_decode_case(name, seed=seed, device="cuda")
        B, hq, d = c["q"].shape
        gate = torch.randn(B, hq, 2 * d, device="cuda", generator=g).to(torch.bfloat16)[..., d:]
        q4, out = c["q"].unsqueeze(1), torch.empty(B, 1, hq, d, dtype=torch.bfloat16, device="cuda")
        args = (q4, c["k_cache"], c["v_cache"], c["context_lens"], c["block_tables"], c["scale"])
        ms_plain = _events_time(lambda i: kernels.paged_decode(*args, out=out), steps, max(warmup, 50))
        ms_gated = _events_time(lambda i: kernels.paged_decode(*args, out=out, gate=gate), steps, max(warmup, 50))
        return dict(ms_per_step=ms_gated, decode_ms=ms_plain, gated_decode_ms=ms_gated,
                    overhead_frac=ms_gated / ms_plain - 1), c
    c = make_prefill_case(name, seed=seed, device="cuda")
    tq, hq, d = c["q"].shape
    out = torch.empty(tq, hq, d, device="cuda", dtype=torch.bfloat16)
    gate = torch.randn(tq, hq, 2 * d, device="cuda", generator=g).to(torch.bfloat16)[..., d:]
    kernels.store_kvcache(c["k_new"], c["v_new"], c["k_cache"], c["v_cache"], c["slot_mapping"])
    args = (c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"], c["cu_seqlens_k"], c["max_seqlen_q"],
            c["max_seqlen_k"], c["scale"])
    kw = dict(block_table=c["block_tables"], out=out)
    ms_plain = _events_time(lambda i: kernels.varlen_prefill(*args, **kw), steps, max(warmup, 10))
    ms_gated = _events_time(lambda i: kernels.varlen_prefill(*args, gate=gate, **kw), steps, max(warmup, 10))
    ms_pass = _events_time(lambda i: kernels.output_gate(out, gate), steps, max(warmup, 200))
    nb = 3 * out.numel() * 2
    return dict(ms_per_step=ms_gated, prefill_ms=ms_plain, gated_prefill_ms=ms_gated,
                fused_overhead_frac=ms_gated / ms_plain - 1, gate_pass_ms=ms_pass,
                gate_pass_gbs=nb / (ms_pass * 1e-3) / 1e9, gate_pass_overhead_frac=ms_pass / ms_plain), c


def bench_gdn(steps, warmup, seed=0, B=64, H=16, HV=32):
    """Gated DeltaNet decode step for a batch of B sequences (Qwen3.5-style
    linear-attention heads: H key heads, HV value heads, K = V = 128, float32
    state pool).  HBM-bound: each (sequence, value head) state is read and
    written once.  The steps rotate over 8 disjoint batches of slots of a
    1 GiB pool, so no step finds the states of an earlier one in the 256 MB
    last-level cache (a model's other layers would evict them)."""
    import torch
    from nano_qwen_amd import kernels

    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=g)
    q, k = r(B, H, 128).bfloat16(), r(B, H, 128).bfloat16()
    v, a, b = r(B, HV, 128).bfloat16(), r(B, HV).bfloat16(), r(B, HV).bfloat16()
    A_log, dt = r(HV) * 0.5, r(HV) * 0.5
    R = 8
    state = r(R * B, HV, 128, 128) * 0.05
    perm = torch.randperm(R * B, device="cuda", generator=g).to(torch.int32)
    idx = [perm[j * B:(j + 1) * B] for j in range(R)]
    out = torch.empty(B, HV, 128, dtype=torch.bfloat16, device="cuda")
    ms = _events_time(lambda i: kernels.gdn_decode(q, k, v, a, b, A_log, dt, state, idx[i % R], out=out),
                      steps, max(warmup, 50))
    nb = 2 * B * HV * 128 * 128 * 4 + (2 * B * H * 128 + 2 * B * HV * 128 + 2 * B * HV) * 2 + B * 4
    return dict(ms_per_step=ms, gbs=nb / (ms * 1e-3) / 1e9, hbm_frac=nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                bytes=nb, batch=B, k_heads=H, v_heads=HV), None


def bench_gdn_prefill(steps, warmup, seed=0, H=16, HV=32):
    """Gated DeltaNet prefill (chunked WY form on MFMA) over cfg3's sequence
    lengths (16 sequences, Lq ~ U[256, 2048]): one 4-wave workgroup per
    (sequence, value head) walks its 64-token chunks.  Reported: tokens/s and
    the rate of the chunked form's nominal product work -- per chunk and
    value head K K^T, Q K^T, P D (64x64x128 each), K S^T, Q S^T
    (64x128x128), the update from V and Y (2 x 64x128x64) and the state
    update (128x128x64): 11 x 64x64x128 multiply-adds, counted over padded
    chunks (the kernel skips the blocks above the diagonal and solves for the
    update blockwise, so it executes less)."""
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import make_prefill_case

    lq = make_prefill_case("cfg3", seed=seed, device="cpu")["lq"]
    cu = torch.tensor([0] + list(torch.tensor(lq).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    T = int(cu[-1])
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=g)
    q, k = r(T, H, 128).bfloat16(), r(T, H, 128).bfloat16()
    v, a, b = r(T, HV, 128).bfloat16(), r(T, HV).bfloat16(), r(T, HV).bfloat16()
    A_log, dt = r(HV) * 0.5, r(HV) * 0.5
    n = len(lq)
    state = torch.zeros(n, HV, 128, 128, device="cuda")
    idx = torch.arange(n, dtype=torch.int32, device="cuda")
    out = torch.empty(T, HV, 128, dtype=torch.bfloat16, device="cuda")
    ms = _events_time(lambda i: kernels.gdn_prefill(q, k, v, a, b, A_log, dt, cu, state, idx, out=out),
                      steps, max(warmup, 3))
    chunks = sum((int(x) + 63) // 64 for x in lq)
    fl = 2.0 * 11 * 64 * 64 * 128 * chunks * HV
    return dict(ms_per_step=ms, tokens=T, tokens_per_s=T / (ms * 1e-3), chunks=chunks,
                mfma_tflops=fl / (ms * 1e-3) / 1e12, mfma_frac=fl / (ms * 1e-3) / 1e12 / 2500.0, k_heads=H,
                v_heads=HV), None


def bench_gated_norm(steps, warmup, seed=0, HV=32):
    """GDN output gated RMS norm over cfg3's token count x HV value heads
    (rows of 128), in place: reads x and the gate, writes x."""
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import make_prefill_case

    T = sum(make_prefill_case("cfg3", seed=seed, device="cpu")["lq"])
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(T, HV, 128, device="cuda", generator=g).bfloat16()
    z = torch.randn(T, HV, 128, device="cuda", generator=g).bfloat16()
    w = torch.rand(128, device="cuda", generator=g) + 0.5
    ms = _events_time(lambda i: kernels.gated_rmsnorm(x, z, w, 1e-6, out=x), steps, max(warmup, 200))
    nb = 3 * x.numel() * 2 + 128 * 4
    return dict(ms_per_step=ms, gbs=nb / (ms * 1e-3) / 1e9, hbm_frac=nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                bytes=nb, rows=T * HV), None


def bench_gdn_conv(steps, warmup, seed=0, C=8192, K=4):
    """GDN causal conv1d + silu over cfg3's packed sequences (prefill) with
    Qwen3.5-style channels C = 2 * 16 * 128 + 32 * 128: reads x once, writes
    the output and each sequence's last K - 1 inputs."""
    import torch
    from nano_qwen_amd import kernels
    from oracle.inputs import make_prefill_case

    lq = make_prefill_case("cfg3", seed=seed, device="cpu")["lq"]
    cu = torch.tensor([0] + list(torch.tensor(lq).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    T = int(cu[-1])
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(T, C, device="cuda", generator=g).bfloat16()
    w = torch.randn(C, K, device="cuda", generator=g).bfloat16()
    state = torch.zeros(len(lq), C, K - 1, device="cuda", dtype=torch.bfloat16)
    idx = torch.arange(len(lq), dtype=torch.int32, device="cuda")
    out = torch.empty_like(x)
    ms = _events_time(lambda i: kernels.gdn_conv1d(x, w, state, idx, cu_seqlens=cu, out=out), steps,
                      max(warmup, 100))
    nb = 2 * x.numel() * 2 + w.numel() * 2 + state.numel() * 2
    return dict(ms_per_step=ms, gbs=nb / (ms * 1e-3) / 1e9, hbm_frac=nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                bytes=nb, tokens=T, channels=C), None


def cpu_baseline_decode(case, n_seqs=8, reps=5):
    """Median wall time of the CPU path on the first n_seqs sequences."""
    import torch
    from oracle import sdpa_path
    from oracle.inputs import decode_bytes

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ids = list(range(n_seqs))
    bs = case["block_size"]
    ctx = case["context_lens"][:n_seqs].cpu()
    nblk = [(int(c) + bs - 1) // bs for c in ctx]
    blocks = torch.cat([case["block_tables"][i, :nblk[i]].long() for i in ids])
    kc = case["k_cache"].index_select(0, blocks.to(case["k_cache"].device)).cpu()
    vc = case["v_cache"].index_select(0, blocks.to(case["v_cache"].device)).cpu()
    bt = torch.full((n_seqs, max(nblk)), -1, dtype=torch.int32)
    off = 0
    for i in ids:
        bt[i, :nblk[i]] = torch.arange(off, off + nblk[i], dtype=torch.int32)
        off += nblk[i]
    slot = torch.tensor([int(bt[i, (int(ctx[i]) - 1) // bs]) * bs + (int(ctx[i]) - 1) % bs for i in ids],
                        dtype=torch.int32)
    q = case["q"][:n_seqs].cpu()
    kn, vn = case["k_new"][:n_seqs].cpu(), case["v_new"][:n_seqs].cpu()
    ks = None if case["k_scale"] is None else case["k_scale"].cpu()
    vs = None if case["v_scale"] is None else case["v_scale"].cpu()

    def run():
        sdpa_path.store_kvcache(kn, vn, kc, vc, slot, ks, vs)
        sdpa_path.paged_decode(q, kc, vc, bt, ctx, case["scale"], ks, vs)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    sub = dict(case, batch=n_seqs, context_lens=ctx, q=q)
    nbytes = decode_bytes(sub)
    return dict(value=nbytes / t / 1e9, unit="GB/s", cores=cores, kind="port",
                sample=f"{case['name']} first {n_seqs} of {case['batch']} sequences (sum ctx "
                       f"{int(ctx.sum())}), store + decode, torch {torch.__version__} CPU, median of {reps}",
                seconds=t, cpu=cpu_model())


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else the platform's."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline_prefill(case, n_seqs=2, reps=3):
    import torch
    from oracle import sdpa_path
    from oracle.inputs import prefill_flops

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ids = list(range(n_seqs))
    lq, lk = case["lq"][:n_seqs], case["lk"][:n_seqs]
    cq = torch.tensor([0] + list(torch.tensor(lq).cumsum(0).tolist()), dtype=torch.int32)
    ck = torch.tensor([0] + list(torch.tensor(lk).cumsum(0).tolist()), dtype=torch.int32)
    bs = case["block_size"]
    nblk = [(x + bs - 1) // bs for x in lk]
    blocks = torch.cat([case["block_tables"][i, :nblk[i]].long() for i in ids])
    kc = case["k_cache"].index_select(0, blocks.to(case["k_cache"].device)).cpu()
    vc = case["v_cache"].index_select(0, blocks.to(case["v_cache"].device)).cpu()
    bt = torch.full((n_seqs, max(nblk)), -1, dtype=torch.int32)
    off = 0
    for i in ids:
        bt[i, :nblk[i]] = torch.arange(off, off + nblk[i], dtype=torch.int32)
        off += nblk[i]
    q = case["q"][: int(cq[-1])].cpu()

    def run():
        sdpa_path.varlen_prefill(q, kc, vc, cq, ck, case["scale"], block_tables=bt)

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    fl = prefill_flops(dict(case, lq=lq, lk=lk))
    return dict(value=fl / t / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                sample=f"{case['name']} first {n_seqs} of {case['nseq']} sequences (Lq {lq}, Lk {lk}), "
                       f"attention only, median of {reps}", seconds=t, cpu=cpu_model())


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "paged_decode_cfg2_traffic.md")


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of the headline kernels and the commit they were
    measured at, from the committed rocprofv3 counter summary (lines
    `traffic_bytes_per_launch: N` and `measured_at_commit: H`), or (None, None)."""
    n = commit = None
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    n = int(line.split(":", 1)[1].strip())
                elif line.strip().startswith("measured_at_commit:"):
                    commit = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return n, commit


def copy_calibration(nbytes, reps=3):
    """A plain device copy of `nbytes` (reads nbytes, writes nbytes), for
    scaling rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch
    x = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "reps": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default=None,
                    help="run one config (cfg2|cfg3|cfg4|cfg5|cfg3_norm_rope|cfg2_norm_rope|cfg2_gate|cfg3_gate|"
                         "cfg2_d256|cfg5_d256|cfg3_d256|gdn_decode|gdn_prefill|gdn_norm|gdn_conv|cfg3_fp8|cfg3_long)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures the paged attention path on ONE GPU; "
              "multi-GPU runs are not part of it (the kernels shard by kv head or by sequence with no communication)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from nano_qwen_amd._lib import lib
    lib()
    torch.cuda.set_device(0)

    extra = {}
    head = None
    todo = [args.only] if args.only else ["cfg2", "cfg3", "cfg4", "cfg5", "cfg3_norm_rope", "cfg2_norm_rope",
                                                   "cfg2_gate", "cfg3_gate", "cfg2_d256", "cfg5_d256",
                                                   "cfg3_d256", "gdn_decode", "gdn_prefill", "gdn_norm",
                                                   "gdn_conv", "cfg3_fp8", "cfg3_long"]
    cpu = None
    for name in todo:
        print(f"[bench] {name} ...", file=sys.stderr, flush=True)
        if name.endswith("_norm_rope"):
            r, case = bench_norm_rope(name.split("_")[0], args.steps, args.warmup)
        elif name.endswith("_gate"):
            r, case = bench_gate(name.split("_")[0], args.steps, args.warmup)
        elif name == "gdn_decode":
            r, case = bench_gdn(args.steps, args.warmup)
        elif name == "gdn_conv":
            r, case = bench_gdn_conv(args.steps, args.warmup)
        elif name == "gdn_norm":
            r, case = bench_gated_norm(args.steps, args.warmup)
        elif name == "gdn_prefill":
            r, case = bench_gdn_prefill(args.steps, args.warmup)
        elif name == "cfg3_fp8":
            r, case = bench_prefill("cfg3", args.steps, args.warmup, kv="fp8")
        elif name == "cfg3_d256":
            r, case = bench_prefill("cfg3", args.steps, args.warmup, d=256, hq=16, hkv=4)
        elif name == "cfg3_long":
            # the same kernel and paged path on long sequences (4 x 8192 new
            # tokens, half with a prefix): few item transitions per product
            r, case = bench_prefill("cfg3", args.steps, args.warmup, nseq=4, lq=(8192, 8192))
        elif name.endswith("_d256"):
            # head_dim 256 (Qwen3.5's full-attention layers) with cfg2's / cfg5's
            # KV bytes per token: Hkv * D = 4 * 256
            r, case = bench_decode(name.split("_")[0], args.steps, args.warmup, d=256, hq=16, hkv=4)
        elif name == "cfg3":
            r, case = bench_prefill(name, args.steps, args.warmup)
            if not args.no_cpu:
                r["cpu_baseline"] = cpu_baseline_prefill(case)
        else:
            r, case = bench_decode(name, args.steps, args.warmup)
            if name == "cfg2":
                head = r
                if not args.no_cpu:
                    cpu = cpu_baseline_decode(case)
        extra[name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        print(f"[bench] {name}: {json.dumps(extra[name])}", file=sys.stderr, flush=True)
        del case
        torch.cuda.empty_cache()

    if head is None:  # --only on a non-headline config: report it as the line
        name = todo[0]
        r = extra[name]
        head_ms = r["ms_per_step"]
        value = (r.get("gbs") or 0.0) if name != "cfg3" else r["tflops"]
        unit = "GB/s" if name != "cfg3" else "TFLOP/s"
    else:
        head_ms, value, unit = head["ms_per_step"], head["gbs"], "GB/s"
    line = {
        "metric": "decode attn HBM GB/s (% of 8 TB/s) + prefill attn TFLOP/s, Qwen3-8B shape",
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V pools, random block permutation)",
        "config": {
            "workload": "cfg2: Qwen3-8B-shaped bf16 paged decode step (store_kvcache + decode), B=64, "
                        "ctx U[1024,4096], Hq=32, Hkv=8, D=128, block_size=256",
            "batch": 64, "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128, "block_size": 256,
        },
    }
    if head is not None:
        line["roofline"] = {
            "bound": "hbm", "kernel": "paged_decode with the fused store (main + split-K merge)",
            "achieved": round(head["step_median_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(head["step_median_gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic()[0],
            "traffic_measured_at_commit": measured_traffic()[1],
            "step_ms": round(head["ms_median"], 5), "algorithmic_bytes": head["bytes_per_step"],
        }
    if "cfg3" in extra:
        line["prefill_tflops"] = extra["cfg3"]["attn_tflops"]
        line["prefill_mfma_frac"] = extra["cfg3"]["mfma_frac"]
    line["cpu_baseline"] = cpu
    line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
