"""MI355X (gfx950) paged-KV attention: the attention hot path of nanovllm_self
rebuilt on hand-written HIP kernels behind the reference's PagedAttention API."""
from .layers.attention import Attention, PagedAttention, reserve_attention_workspace
from .utils.context import Context, get_context

__all__ = ["Attention", "PagedAttention", "Context", "get_context", "reserve_attention_workspace"]
