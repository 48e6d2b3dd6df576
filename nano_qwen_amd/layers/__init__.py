from .attention import Attention, store_kvcache
from .gated_delta_net import gdn_core
from .qk_norm_rope import qk_norm_rope_store

__all__ = ["Attention", "store_kvcache", "qk_norm_rope_store", "gdn_core"]
