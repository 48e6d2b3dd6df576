"""MI355X (gfx950) paged attention path for nano_qwen.

A drop-in for the reference's paged attention path: ``layers.Attention`` and
``layers.store_kvcache`` keep the reference's contract
(layers/attention.py:33-75), ``utils.context`` keeps its ``Context`` fields
and ``engine.ModelRunner`` restates ``prepare_prefill`` / ``prepare_decode``;
the device work runs in hand-written HIP kernels (``libnq_attn.so``, C ABI in
``include/nq_attn.h``) reached through ``kernels``.
"""
from . import kernels
from .layers import Attention, store_kvcache
from .utils.context import Context, get_context, reset_context, set_context

__all__ = ["Attention", "store_kvcache", "kernels", "Context", "get_context", "set_context",
           "reset_context"]
__version__ = "0.1.0"
