"""The HIP kernels against the committed golden fixtures (tests/golden/).

Inputs are loaded from the fixtures (so the GPU box needs nothing else) and
the outputs compared with the stored float64-oracle expectations: bf16
attention within the bf16 tolerance, the fp8 store byte for byte.
"""
import os

import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from tests.parity import TOL_BF16, assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16(u16, dev):
    return torch.from_numpy(u16.view(np.int16).copy()).view(torch.bfloat16).to(dev)


def test_golden_decode_gpu(cuda):
    z = load("decode_bf16_small.npz")
    print("[golden] decode_bf16_small", flush=True)
    out = kernels.paged_decode(bf16(z["q"], cuda).unsqueeze(1), bf16(z["k_cache"], cuda), bf16(z["v_cache"], cuda),
                               torch.from_numpy(z["context_lens"]).to(cuda),
                               torch.from_numpy(z["block_tables"]).to(cuda), float(z["scale"]))
    torch.cuda.synchronize()
    assert_close(out[:, 0].double().cpu().numpy(), z["out"].astype(np.float64), **TOL_BF16, what="golden decode")


def test_golden_prefill_gpu(cuda):
    z = load("prefill_bf16_paged_small.npz")
    print("[golden] prefill_bf16_paged_small", flush=True)
    cu_q, cu_k = z["cu_seqlens_q"], z["cu_seqlens_k"]
    out = kernels.varlen_prefill(bf16(z["q"], cuda), bf16(z["k_cache"], cuda), bf16(z["v_cache"], cuda),
                                 torch.from_numpy(cu_q).to(cuda), torch.from_numpy(cu_k).to(cuda),
                                 int(np.diff(cu_q).max()), int(np.diff(cu_k).max()), float(z["scale"]),
                                 causal=True, block_table=torch.from_numpy(z["block_tables"]).to(cuda))
    torch.cuda.synchronize()
    assert_close(out.double().cpu().numpy(), z["out"].astype(np.float64), **TOL_BF16, what="golden prefill")


def test_golden_store_fp8_gpu(cuda):
    z = load("store_fp8_small.npz")
    print("[golden] store_fp8_small", flush=True)
    kc = torch.zeros(z["k_cache"].shape, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    vc = torch.zeros(z["v_cache"].shape, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    kernels.store_kvcache(bf16(z["key"], cuda), bf16(z["value"], cuda), kc, vc,
                          torch.from_numpy(z["slot_mapping"]).to(cuda), torch.from_numpy(z["k_scale"]).to(cuda),
                          torch.from_numpy(z["v_scale"]).to(cuda))
    torch.cuda.synchronize()
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), z["k_cache"])
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), z["v_cache"])
