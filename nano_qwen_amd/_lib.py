"""ctypes binding of libnq_attn.so (the C ABI declared in include/nq_attn.h).

torch is imported first so that the HIP runtime torch loaded is the one the
library binds to (one runtime per process; torch's device pointers and
streams are then valid in the library).  There is no fallback: if the
library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p, POINTER
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libnq_attn.so")

NQ_F32, NQ_F16, NQ_BF16, NQ_FP8_E4M3 = 0, 1, 2, 3
DTYPES = {
    torch.float32: NQ_F32,
    torch.float16: NQ_F16,
    torch.bfloat16: NQ_BF16,
    torch.float8_e4m3fn: NQ_FP8_E4M3,
}

# name -> (restype, argtypes); must match include/nq_attn.h
_SIGS = {
    "nq_abi_version": (c_int, []),
    "nq_last_error": (ctypes.c_char_p, []),
    "nq_store_kvcache": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                 c_int64, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                 c_void_p]),
    "nq_decode_plan": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, POINTER(c_int), POINTER(c_int)]),
    "nq_decode_workspace_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "nq_decode_schedule": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int64]),
    "nq_paged_decode": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int,
                                c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int,
                                c_int64, c_float, c_int, c_int, c_void_p, c_int64, c_int, c_int, c_void_p,
                                c_void_p, c_void_p]),
    "nq_paged_decode_gated": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                      c_int, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int,
                                      c_int, c_int64, c_float, c_int, c_int, c_void_p, c_int64, c_int, c_int,
                                      c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "nq_paged_decode_store": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                      c_int, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int,
                                      c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int,
                                      c_int, c_int64, c_float, c_int, c_int, c_void_p, c_int64, c_int, c_int,
                                      c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "nq_paged_decode_noalloc": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int,
                                        c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int,
                                        c_int64, c_float, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                        c_void_p]),
    "nq_output_gate": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int, c_int,
                               c_int, c_void_p]),
    "nq_varlen_prefill": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                                  c_void_p, c_int, c_int, c_void_p, c_int64, c_int, c_int64, c_void_p,
                                  c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                  c_int, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "nq_varlen_prefill_gated": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                                        c_void_p, c_int, c_int, c_void_p, c_int64, c_int, c_int64, c_void_p,
                                        c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                        c_int, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
                                        c_int64, c_int64, c_void_p]),
    "nq_prefill_workspace_bytes": (c_int64, []),
    "nq_prepare_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_int, c_int, c_void_p]),
    "nq_gdn_decode": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                              c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                              c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "nq_gdn_prefill": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                               c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                               c_int64, c_int, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "nq_gated_rmsnorm": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_float, c_void_p, c_int64,
                                 c_int64, c_int, c_int, c_void_p]),
    "nq_gdn_conv1d": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_int64,
                              c_int, c_void_p, c_int64, c_int, c_int, c_void_p]),
    "nq_qk_norm_rope_store": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                      c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_float,
                                      c_float, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                      c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int,
                                      c_int, c_void_p, c_void_p, c_void_p]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built: run `python -m nano_qwen_amd.build` "
                "(the HIP kernels have no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.nq_abi_version() != 1:
            raise RuntimeError(f"{LIB_PATH.name}: ABI version {handle.nq_abi_version()} != 1")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().nq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def dtype_code(t: torch.dtype) -> int:
    try:
        return DTYPES[t]
    except KeyError:
        raise RuntimeError(f"dtype {t} is not supported by the HIP kernels") from None


def ptr(t):
    return None if t is None else c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor) -> c_void_p:
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*tensors, what: str) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{what}: tensors must be on a HIP device (got {t.device}); "
                               "this path has no CPU implementation")
