"""Aligned record files of the page stores.

The on-disk contract is the reference's (src/seqattn_core/storage/direct_io.py:
records at 4,096-byte aligned offsets and lengths, O_DIRECT optional, a JSON
manifest published atomically).  The machinery is this package's own:

* ``RecordFile`` owns one descriptor and moves whole byte ranges with
  ``preadv``/``pwritev``, reporting short transfers and O_DIRECT refusals.
* ``PageBuffer`` is a page-aligned anonymous mapping (the only kind of host
  memory O_DIRECT accepts here besides page-locked slots) with a uint8
  tensor view for staging tensors in and out.
* ``BufferPool`` lends a fixed set of page buffers to concurrent I/O threads
  and charges them to the ``bounce`` category of a host-memory plan for as
  long as it lives.

Buffered stores do not need the bounce buffers at all: their readers and
writers move rows straight between the file and the caller's tensors.
"""

from __future__ import annotations

import errno
import json
import mmap
import os
import threading
from contextlib import contextmanager
from pathlib import Path

import torch

DIRECT_IO_ALIGNMENT = 4096
FORMAT_VERSION = 1
# errno values with which a filesystem refuses O_DIRECT opens or transfers.
_DIRECT_REFUSALS = frozenset({errno.EINVAL, errno.EOPNOTSUPP, errno.ENOTSUP})


def round_up(value: int, alignment: int = DIRECT_IO_ALIGNMENT) -> int:
    return -(-value // alignment) * alignment


def open_file(path: Path, flags: int, mode: int, direct_io: bool) -> int:
    """``os.open`` with O_DIRECT added when asked.  A filesystem that refuses
    O_DIRECT raises RuntimeError; there is no silent buffered fallback."""
    if direct_io:
        o_direct = getattr(os, "O_DIRECT", None)
        if o_direct is None:
            raise RuntimeError("O_DIRECT is unavailable on this platform")
        flags |= o_direct
    try:
        return os.open(path, flags, mode)
    except OSError as error:
        if direct_io and error.errno in _DIRECT_REFUSALS | {errno.ENODEV}:
            raise RuntimeError(f"filesystem does not support required O_DIRECT access for {path}") from error
        raise


def byte_view(tensor: torch.Tensor) -> memoryview:
    """Writable memoryview over a contiguous CPU tensor's bytes."""
    return memoryview(tensor.view(torch.uint8).reshape(-1).numpy())


class RecordFile:
    """One store file, opened for whole-range reads or writes."""

    def __init__(self, path: Path, *, write: bool, direct_io: bool) -> None:
        self.path = Path(path)
        self.direct_io = direct_io
        flags = os.O_CREAT | os.O_TRUNC | os.O_WRONLY if write else os.O_RDONLY
        self.fd = open_file(self.path, flags, 0o644, direct_io)

    def _transfer(self, call, buffers: list[memoryview], offset: int, what: str) -> None:
        wanted = sum(len(b) for b in buffers)
        try:
            moved = call(self.fd, buffers, offset)
        except OSError as error:
            if self.direct_io and error.errno in _DIRECT_REFUSALS:
                raise RuntimeError(f"filesystem rejected required O_DIRECT {what} for {self.path}") from error
            raise
        if moved != wanted:
            preposition = "from" if what == "read" else "to"
            raise OSError(errno.EIO, f"short {what}: {moved} != {wanted} {preposition} {self.path}")

    def read_into(self, offset: int, *buffers: memoryview) -> None:
        """Fill ``buffers`` (in order) from the file bytes at ``offset``."""
        self._transfer(os.preadv, list(buffers), offset, "read")

    def write_from(self, offset: int, *buffers: memoryview) -> None:
        """Write ``buffers`` (in order) at ``offset``; the range must be aligned."""
        length = sum(len(b) for b in buffers)
        if offset % DIRECT_IO_ALIGNMENT or length % DIRECT_IO_ALIGNMENT:
            raise ValueError("direct-I/O writes must use 4096-byte aligned offsets and lengths")
        self._transfer(os.pwritev, list(buffers), offset, "write")

    def close(self, *, sync: bool = False) -> None:
        if self.fd < 0:
            return
        fd, self.fd = self.fd, -1
        try:
            if sync:
                os.fsync(fd)
        finally:
            os.close(fd)


class PageBuffer:
    """Page-aligned anonymous mapping with a uint8 tensor view over it."""

    def __init__(self, size_bytes: int) -> None:
        self.size_bytes = round_up(max(size_bytes, 1))
        self._mapping = mmap.mmap(-1, self.size_bytes, access=mmap.ACCESS_WRITE)
        self.bytes = torch.frombuffer(self._mapping, dtype=torch.uint8, count=self.size_bytes)

    def window(self, size_bytes: int) -> memoryview:
        return memoryview(self._mapping)[:size_bytes]

    def put(self, offset: int, tensor: torch.Tensor) -> None:
        """Copy a CPU tensor's bytes into the buffer at ``offset``."""
        flat = tensor.detach().contiguous().view(torch.uint8).reshape(-1)
        if offset + flat.numel() > self.size_bytes:
            raise ValueError("tensor does not fit in the aligned bounce buffer")
        self.bytes[offset : offset + flat.numel()].copy_(flat)

    def get(self, offset: int, out: torch.Tensor, elements: int) -> None:
        """Copy ``elements`` items of ``out``'s dtype from ``offset`` into ``out``."""
        count = elements * out.element_size()
        out.reshape(-1)[:elements].view(torch.uint8).copy_(self.bytes[offset : offset + count])

    def release(self) -> None:
        self.bytes = torch.empty(0, dtype=torch.uint8)
        self._mapping.close()


class BufferPool:
    """``count`` page buffers of ``size_bytes`` lent to one I/O thread at a time.

    The buffers are charged to ``memory_plan``'s ``bounce`` category (when a
    plan is given) until ``close``.
    """

    def __init__(self, count: int, size_bytes: int, memory_plan=None) -> None:
        self._buffers = [PageBuffer(size_bytes) for _ in range(max(1, count))]
        self.charged_bytes = sum(b.size_bytes for b in self._buffers)
        self._plan = memory_plan
        if memory_plan is not None:
            try:
                memory_plan.register("bounce", self.charged_bytes)
            except BaseException:
                self._drop()
                raise
        self._idle = list(self._buffers)
        self._ready = threading.Condition()

    @contextmanager
    def lease(self):
        with self._ready:
            while not self._idle:
                self._ready.wait()
            buffer = self._idle.pop()
        try:
            yield buffer
        finally:
            with self._ready:
                self._idle.append(buffer)
                self._ready.notify()

    def _drop(self) -> None:
        for buffer in self._buffers:
            buffer.release()
        self._buffers = []

    def close(self) -> None:
        if not self._buffers:
            return
        if self._plan is not None:
            self._plan.release("bounce", self.charged_bytes)
        self._drop()


def sync_directory(path: Path) -> None:
    fd = os.open(path, os.O_RDONLY | getattr(os, "O_DIRECTORY", 0))
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def publish_json(path: Path, payload: dict[str, object]) -> None:
    """Write ``payload`` to ``path`` so that readers see either nothing or the
    whole file: a synced temporary renamed into place, then the directory
    synced."""
    staged = path.with_suffix(path.suffix + ".tmp")
    data = (json.dumps(payload, indent=2, sort_keys=True) + "\n").encode("utf-8")
    with open(staged, "wb") as handle:
        handle.write(data)
        handle.flush()
        os.fsync(handle.fileno())
    os.replace(staged, path)
    sync_directory(path.parent)


__all__ = [
    "DIRECT_IO_ALIGNMENT",
    "FORMAT_VERSION",
    "BufferPool",
    "PageBuffer",
    "RecordFile",
    "byte_view",
    "open_file",
    "publish_json",
    "round_up",
    "sync_directory",
]
