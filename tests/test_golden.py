"""The CPU oracle reproduces the committed golden fixtures (tests/golden/).

The fixtures were written by tests/golden/make_golden.py from the float64
oracle; re-deriving them here pins the oracle against silent changes.  The
fp8 store is compared byte for byte; attention outputs to float32 rounding.
"""
import os

import numpy as np
import torch

from oracle import fp8, paged

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def f64_from_bits(u16):
    return torch.from_numpy(u16.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()


def test_golden_decode_oracle():
    z = load("decode_bf16_small.npz")
    out = paged.paged_decode(f64_from_bits(z["q"]), f64_from_bits(z["k_cache"]), f64_from_bits(z["v_cache"]),
                             z["block_tables"], z["context_lens"].astype(np.int64), float(z["scale"]))
    np.testing.assert_allclose(out, z["out"], rtol=1e-6, atol=1e-6)
    # context 1: the output is exactly the first cached V row of the block
    v = f64_from_bits(z["v_cache"])
    blk = int(z["block_tables"][0, 0])
    g = z["q"].shape[1] // v.shape[2]
    for h in range(z["q"].shape[1]):
        np.testing.assert_allclose(z["out"][0, h], v[blk, 0, h // g], rtol=1e-6, atol=1e-6)


def test_golden_prefill_oracle():
    z = load("prefill_bf16_paged_small.npz")
    out = paged.varlen_prefill(f64_from_bits(z["q"]), f64_from_bits(z["k_cache"]), f64_from_bits(z["v_cache"]),
                               z["cu_seqlens_q"], z["cu_seqlens_k"], float(z["scale"]),
                               block_tables=z["block_tables"])
    np.testing.assert_allclose(out, z["out"], rtol=1e-6, atol=1e-6)


def test_golden_store_fp8_oracle():
    z = load("store_fp8_small.npz")
    key = f64_from_bits(z["key"]).astype(np.float32)
    value = f64_from_bits(z["value"]).astype(np.float32)
    kc = np.zeros_like(z["k_cache"])
    vc = np.zeros_like(z["v_cache"])
    paged.store_kvcache(fp8.quantize(key, z["k_scale"]), fp8.quantize(value, z["v_scale"]), kc, vc,
                        z["slot_mapping"])
    assert np.array_equal(kc, z["k_cache"]) and np.array_equal(vc, z["v_cache"])
    # the skipped token (slot -1) left no trace; saturation happened
    assert (z["k_cache"] == 0x7E).any() and (z["k_cache"] == 0xFE).any()
