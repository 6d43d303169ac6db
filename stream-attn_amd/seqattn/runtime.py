"""Import path of the streaming runner kept from the reference (src/seqattn/runtime.py)."""

from .streaming import StreamingAttentionRunner, resolve_backend

__all__ = ["StreamingAttentionRunner", "resolve_backend"]
