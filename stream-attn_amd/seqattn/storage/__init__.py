"""Aligned on-disk page stores (reference src/seqattn_core/storage/__init__.py)."""

from .direct_io import DIRECT_IO_ALIGNMENT
from .output import NvmeOutputSink, ephemeral_nvme_directory, load_nvme_output
from .qkv_store import NvmeQKVStore
from .qkv_writer import NvmeQKVWriter

__all__ = [
    "DIRECT_IO_ALIGNMENT",
    "NvmeOutputSink",
    "NvmeQKVStore",
    "NvmeQKVWriter",
    "ephemeral_nvme_directory",
    "load_nvme_output",
]
