"""Import path of the paged runner kept from the reference (src/seqattn/paged_runtime.py)."""

from .paged.runtime import PagedAttentionRunner

__all__ = ["PagedAttentionRunner"]
