from .context import Context, get_context

__all__ = ["Context", "get_context"]
