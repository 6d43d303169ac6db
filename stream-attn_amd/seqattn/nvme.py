"""Import path of the aligned page stores kept from the reference (src/seqattn/nvme.py)."""

from .storage import (
    DIRECT_IO_ALIGNMENT,
    NvmeOutputSink,
    NvmeQKVStore,
    NvmeQKVWriter,
    ephemeral_nvme_directory,
    load_nvme_output,
)

__all__ = [
    "DIRECT_IO_ALIGNMENT",
    "NvmeOutputSink",
    "NvmeQKVStore",
    "NvmeQKVWriter",
    "ephemeral_nvme_directory",
    "load_nvme_output",
]


def _open_file(path, flags, mode, direct_io):
    """Open with O_DIRECT when asked; unsupported O_DIRECT raises (no buffered fallback)."""
    from .storage.direct_io import open_file

    return open_file(path, flags, mode, direct_io)
