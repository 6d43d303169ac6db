"""Import path of page models and in-memory backends kept from the reference (src/seqattn/paging.py)."""

from .paged.layout import (
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
from .paged.memory import CallbackOutputSink, MemoryPageSink, MemoryPageSource
from .paged.protocols import PageReader, PageSink, PageSource, PageWriter

__all__ = [
    "CallbackOutputSink",
    "KVLayout",
    "MemoryPageSink",
    "MemoryPageSource",
    "PageDescriptor",
    "PageReadMetrics",
    "PageReader",
    "PageSink",
    "PageSource",
    "PageWriter",
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
