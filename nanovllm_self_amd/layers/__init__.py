from .attention import Attention, PagedAttention

__all__ = ["Attention", "PagedAttention"]
