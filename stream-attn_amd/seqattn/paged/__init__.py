"""Paged sources, sinks and the paged runner (reference src/seqattn_core/paged/__init__.py)."""

from .cache import CacheLookup, KVPageCache
from .layout import (
    KVLayout,
    PageDescriptor,
    PageReadMetrics,
    TensorLayout,
    align_down,
    align_up,
    build_page_descriptors,
    dtype_name,
    pages_by_segment,
    replace_page,
    torch_dtype,
    validate_cu_seqlens,
)
from .memory import CallbackOutputSink, MemoryPageSink, MemoryPageSource
from .memory_budget import HostMemoryPlan, HostMemorySnapshot
from .protocols import PageReader, PageSink, PageSource, PageWriter
from .runtime import PagedAttentionRunner

__all__ = [
    "CacheLookup",
    "CallbackOutputSink",
    "HostMemoryPlan",
    "HostMemorySnapshot",
    "KVLayout",
    "KVPageCache",
    "MemoryPageSink",
    "MemoryPageSource",
    "PageDescriptor",
    "PageReadMetrics",
    "PageReader",
    "PageSink",
    "PageSource",
    "PageWriter",
    "PagedAttentionRunner",
    "TensorLayout",
    "align_down",
    "align_up",
    "build_page_descriptors",
    "dtype_name",
    "pages_by_segment",
    "replace_page",
    "torch_dtype",
    "validate_cu_seqlens",
]
