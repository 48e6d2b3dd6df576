from .attention import Attention, store_kvcache

__all__ = ["Attention", "store_kvcache"]
