"""store_kvcache on the GPU vs the oracle: bit-exact (layers/attention.py:10-40)."""
import numpy as np
import pytest
import torch

from nano_qwen_amd import kernels
from nano_qwen_amd.layers import store_kvcache
from oracle import fp8, paged
from oracle.inputs import fp8_scales

pytestmark = pytest.mark.gpu


def _case(dev, dtype, n=37, nb=9, bs=256, hkv=8, d=128, seed=0, skip=(3, 11)):
    g = torch.Generator(device="cpu").manual_seed(seed)
    kc = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    vc = torch.randn(nb, bs, hkv, d, generator=g).to(dtype)
    key = torch.randn(n, hkv, d, generator=g).to(dtype)
    val = torch.randn(n, hkv, d, generator=g).to(dtype)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    for i in skip:
        if i < n:
            slots[i] = -1
    return kc, vc, key, val, slots


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_bit_exact(cuda, dtype):
    kc, vc, key, val, slots = _case(cuda, dtype)
    kn, vn = kc.clone(), vc.clone()
    view = torch.int16 if dtype != torch.float32 else torch.int32
    paged.store_kvcache(key.view(view).numpy(), val.view(view).numpy(), kn.view(view).numpy(),
                        vn.view(view).numpy(), slots.numpy())
    kg, vg = kc.to(cuda), vc.to(cuda)
    store_kvcache(key.to(cuda), val.to(cuda), kg, vg, slots.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(view), kn.view(view))
    assert torch.equal(vg.cpu().view(view), vn.view(view))


def test_store_strided_rows_and_decode_batch(cuda):
    # key rows with a row stride larger than Hkv*D (a view of a wider tensor)
    kc, vc, key, val, slots = _case(cuda, torch.bfloat16, n=64, skip=())
    wide_k = torch.randn(64, 3, 8, 128).to(torch.bfloat16)
    wide_v = torch.randn(64, 3, 8, 128).to(torch.bfloat16)
    wide_k[:, 1] = key
    wide_v[:, 2] = val
    kg, vg = kc.to(cuda), vc.to(cuda)
    wk, wv = wide_k.to(cuda), wide_v.to(cuda)
    store_kvcache(wk[:, 1], wv[:, 2], kg, vg, slots.to(cuda))
    kn, vn = kc.clone(), vc.clone()
    paged.store_kvcache(key.view(torch.int16).numpy(), val.view(torch.int16).numpy(),
                        kn.view(torch.int16).numpy(), vn.view(torch.int16).numpy(), slots.numpy())
    assert torch.equal(kg.cpu().view(torch.int16), kn.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vn.view(torch.int16))


def test_store_all_skipped_and_empty(cuda):
    kc, vc, key, val, slots = _case(cuda, torch.bfloat16, n=5)
    slots[:] = -1
    kg, vg = kc.to(cuda), vc.to(cuda)
    store_kvcache(key.to(cuda), val.to(cuda), kg, vg, slots.to(cuda))
    store_kvcache(key[:0].to(cuda), val[:0].to(cuda), kg, vg, slots[:0].to(cuda))
    assert torch.equal(kg.cpu().view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vc.view(torch.int16))


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_fp8_bit_exact(cuda, in_dtype):
    n, nb, bs, hkv, d = 300, 4, 256, 8, 128
    g = torch.Generator().manual_seed(5)
    # magnitudes spanning e4m3 subnormals to saturation
    mag = torch.tensor([1e-4, 1e-3, 0.02, 1.0, 5.0, 80.0])[torch.randint(0, 6, (n, hkv, 1), generator=g)]
    key = (torch.randn(n, hkv, d, generator=g) * mag).to(in_dtype)
    val = (torch.randn(n, hkv, d, generator=g) * mag).to(in_dtype)
    ks = fp8_scales(key) * 0.5     # some values saturate at +-448
    vs = fp8_scales(val)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[7] = -1
    kc = torch.zeros(nb, bs, hkv, d, dtype=torch.uint8)
    vc = torch.zeros(nb, bs, hkv, d, dtype=torch.uint8)
    kq = fp8.quantize(key.float().numpy(), ks.numpy())
    vq = fp8.quantize(val.float().numpy(), vs.numpy())
    kn, vn = kc.numpy().copy(), vc.numpy().copy()
    paged.store_kvcache(kq, vq, kn, vn, slots.numpy())
    kg = kc.to(cuda).view(torch.float8_e4m3fn)
    vg = vc.to(cuda).view(torch.float8_e4m3fn)
    kernels.store_kvcache(key.to(cuda), val.to(cuda), kg, vg, slots.to(cuda), ks.to(cuda), vs.to(cuda))
    torch.cuda.synchronize()
    kgot = kg.view(torch.uint8).cpu().numpy()
    vgot = vg.view(torch.uint8).cpu().numpy()
    bad = np.argwhere(kgot != kn)
    assert bad.size == 0, f"{len(bad)} K codes differ, first at {bad[:3].tolist()}: got {kgot[tuple(bad[0])]:#x} want {kn[tuple(bad[0])]:#x}"
    assert np.array_equal(vgot, vn)


def test_store_fp8_nan_stays_nan(cuda):
    key = torch.zeros(2, 8, 128)
    key[0, 3, 5] = float("nan")
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ones = torch.ones(8, device=cuda)
    kernels.store_kvcache(key.to(cuda), key.to(cuda), kc, vc, torch.tensor([0, 1], dtype=torch.int32, device=cuda),
                          ones, ones)
    got = kc.float().cpu()
    assert torch.isnan(got[0, 0, 3, 5]) and torch.isfinite(got[0, 1]).all()

