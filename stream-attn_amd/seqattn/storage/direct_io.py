"""Aligned file I/O for page stores (reference src/seqattn_core/storage/direct_io.py:14-152).

Records are written and read whole, at 4,096-byte aligned offsets and
lengths, optionally with O_DIRECT (no page-cache copy).  Buffers handed to
O_DIRECT must be 4,096-byte aligned: anonymous mmaps here, or page-locked
slots of the paged runtime's pinned slab.
"""

from __future__ import annotations

import errno
import json
import mmap
import os
from pathlib import Path

import torch

from ..paged.layout import align_up

DIRECT_IO_ALIGNMENT = 4096
FORMAT_VERSION = 1
_REJECTED = {errno.EINVAL, errno.EOPNOTSUPP, errno.ENOTSUP}


def open_file(path: Path, flags: int, mode: int, direct_io: bool) -> int:
    if direct_io:
        direct = getattr(os, "O_DIRECT", None)
        if direct is None:
            raise RuntimeError("O_DIRECT is unavailable on this platform")
        flags |= direct
    try:
        return os.open(path, flags, mode)
    except OSError as error:
        if direct_io and error.errno in _REJECTED | {errno.ENODEV}:
            raise RuntimeError(f"filesystem does not support required O_DIRECT access for {path}") from error
        raise


def fsync_directory(path: Path) -> None:
    fd = os.open(path, os.O_RDONLY | getattr(os, "O_DIRECTORY", 0))
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def atomic_write_json(path: Path, payload: dict[str, object]) -> None:
    """Write-to-temporary, fsync, rename, fsync the directory."""
    temporary = path.with_suffix(path.suffix + ".tmp")
    data = (json.dumps(payload, indent=2, sort_keys=True) + "\n").encode("utf-8")
    fd = os.open(temporary, os.O_CREAT | os.O_TRUNC | os.O_WRONLY, 0o644)
    try:
        written = os.write(fd, data)
        if written != len(data):
            raise OSError(errno.EIO, f"short manifest write: {written} != {len(data)}")
        os.fsync(fd)
    finally:
        os.close(fd)
    os.replace(temporary, path)
    fsync_directory(path.parent)


def pread_exact(fd: int, buffer: memoryview, offset: int, direct_io: bool, path: Path) -> None:
    """Read exactly len(buffer) bytes at offset."""
    try:
        got = os.preadv(fd, [buffer], offset)
    except OSError as error:
        if direct_io and error.errno in _REJECTED:
            raise RuntimeError(f"filesystem rejected required O_DIRECT read for {path}") from error
        raise
    if got != len(buffer):
        raise OSError(errno.EIO, f"short read: {got} != {len(buffer)} from {path}")


def pwrite_exact(fd: int, buffer: memoryview, offset: int, direct_io: bool, path: Path) -> None:
    """Write exactly len(buffer) bytes at offset."""
    if offset % DIRECT_IO_ALIGNMENT or len(buffer) % DIRECT_IO_ALIGNMENT:
        raise ValueError("direct-I/O writes must use 4096-byte aligned offsets and lengths")
    try:
        put = os.pwritev(fd, [buffer], offset)
    except OSError as error:
        if direct_io and error.errno in _REJECTED:
            raise RuntimeError(f"filesystem rejected required O_DIRECT write for {path}") from error
        raise
    if put != len(buffer):
        raise OSError(errno.EIO, f"short write: {put} != {len(buffer)}")


def byte_view(tensor: torch.Tensor) -> memoryview:
    """Writable memoryview over a contiguous CPU tensor's bytes."""
    return memoryview(tensor.view(torch.uint8).reshape(-1).numpy())


class AlignedBuffer:
    """Page-aligned anonymous mapping used as an O_DIRECT bounce buffer."""

    def __init__(self, size_bytes: int) -> None:
        self.size_bytes = align_up(max(size_bytes, DIRECT_IO_ALIGNMENT), DIRECT_IO_ALIGNMENT)
        self.mapping = mmap.mmap(-1, self.size_bytes, access=mmap.ACCESS_WRITE)
        self.bytes = torch.frombuffer(self.mapping, dtype=torch.uint8, count=self.size_bytes)

    def view(self, size_bytes: int) -> memoryview:
        return memoryview(self.mapping)[:size_bytes]

    def zero(self, size_bytes: int) -> None:
        self.bytes[:size_bytes].zero_()

    def copy_tensor(self, offset: int, tensor: torch.Tensor) -> int:
        src = tensor.detach().contiguous().view(torch.uint8).reshape(-1)
        if offset + src.numel() > self.size_bytes:
            raise ValueError("tensor does not fit in the aligned bounce buffer")
        self.bytes[offset : offset + src.numel()].copy_(src)
        return src.numel()

    def copy_to_tensor(self, offset: int, tensor: torch.Tensor, element_count: int) -> None:
        count = element_count * tensor.element_size()
        tensor.reshape(-1)[:element_count].view(torch.uint8).copy_(self.bytes[offset : offset + count])

    def close(self) -> None:
        self.bytes = torch.empty(0, dtype=torch.uint8)
        self.mapping.close()


class AlignedFileWriter:
    """Whole-record writer of one store file."""

    def __init__(self, path: Path, max_record_bytes: int, direct_io: bool) -> None:
        self.path = path
        self.direct_io = direct_io
        self.fd = open_file(path, os.O_CREAT | os.O_TRUNC | os.O_WRONLY, 0o644, direct_io)
        self.buffer = AlignedBuffer(max_record_bytes)
        self.closed = False

    def write(self, offset: int, storage_bytes: int) -> None:
        view = self.buffer.view(storage_bytes)
        try:
            pwrite_exact(self.fd, view, offset, self.direct_io, self.path)
        finally:
            view.release()

    def close(self) -> None:
        if self.closed:
            return
        try:
            os.fsync(self.fd)
        finally:
            os.close(self.fd)
            self.buffer.close()
            self.closed = True


__all__ = [
    "DIRECT_IO_ALIGNMENT",
    "FORMAT_VERSION",
    "AlignedBuffer",
    "AlignedFileWriter",
    "atomic_write_json",
    "byte_view",
    "fsync_directory",
    "open_file",
    "pread_exact",
    "pwrite_exact",
]
