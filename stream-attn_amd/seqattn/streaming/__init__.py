from .backend import resolve_backend
from .runner import StreamingAttentionRunner

__all__ = ["StreamingAttentionRunner", "resolve_backend"]
