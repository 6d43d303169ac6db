"""Aligned output page store (reference src/seqattn_core/storage/output.py:31-251).

``NvmeOutputSink`` writes every output page as a 4,096-byte aligned record of
a temporary file; ``close`` fsyncs, renames it into place and writes the
manifest last, ``abort`` removes the partial output.  ``load_nvme_output``
reads a finished store back into one tensor.
"""

from __future__ import annotations

import errno
import json
import os
import queue
import shutil
import tempfile
import threading
import time
from collections.abc import Iterator, Sequence
from contextlib import contextmanager
from pathlib import Path

import torch

from ..paged.layout import PageDescriptor, PageReadMetrics, TensorLayout
from ..paged.memory_budget import HostMemoryPlan
from ..paged.protocols import PageSink, PageWriter
from .direct_io import (
    DIRECT_IO_ALIGNMENT,
    FORMAT_VERSION,
    AlignedBuffer,
    atomic_write_json,
    fsync_directory,
    open_file,
    pread_exact,
    pwrite_exact,
)
from .records import expected_file_size, q_record_pages


class _NvmeOutputWriter(PageWriter):
    def __init__(self, sink: NvmeOutputSink, layout: TensorLayout, cu_seqlens: Sequence[int],
                 pages: Sequence[PageDescriptor], memory_plan: HostMemoryPlan, queue_depth: int) -> None:
        self.sink = sink
        self.layout = layout
        self.cu_seqlens = tuple(cu_seqlens)
        self.pages = q_record_pages(pages, layout)
        self.records = {p.page_id: p for p in self.pages}
        self.path = sink.path
        self.path.mkdir(parents=True, exist_ok=True)
        if (self.path / "manifest.json").exists():
            raise FileExistsError(f"output store already exists: {self.path}")
        self.tmp_path = self.path / "out.bin.tmp"
        self.final_path = self.path / "out.bin"
        largest = max((p.storage_bytes for p in self.pages), default=DIRECT_IO_ALIGNMENT)
        self.buffers = [AlignedBuffer(largest) for _ in range(max(1, queue_depth))]
        self.registered_bytes = sum(b.size_bytes for b in self.buffers)
        try:
            memory_plan.register("bounce", self.registered_bytes)
        except BaseException:
            for b in self.buffers:
                b.close()
            raise
        self.memory_plan = memory_plan
        self.free: queue.LifoQueue[AlignedBuffer] = queue.LifoQueue()
        for b in self.buffers:
            self.free.put(b)
        try:
            self.fd = open_file(self.tmp_path, os.O_CREAT | os.O_TRUNC | os.O_WRONLY, 0o644, sink.direct_io)
        except BaseException:
            memory_plan.release("bounce", self.registered_bytes)
            for b in self.buffers:
                b.close()
            raise
        self.closed = False
        self._lock = threading.Lock()

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        record = self.records[page.page_id]
        rows = data[: page.valid_tokens]
        if data.device.type != "cpu" or tuple(rows.shape) != (page.valid_tokens, self.layout.heads,
                                                             self.layout.head_dim):
            raise ValueError("output page tensor does not match its descriptor")
        if data.dtype != self.layout.torch_dtype:
            raise ValueError("output page dtype does not match output layout")
        buffer = self.free.get()
        started = time.perf_counter()
        try:
            buffer.zero(record.storage_bytes)
            buffer.copy_tensor(0, rows)
            view = buffer.view(record.storage_bytes)
            try:
                with self._lock:
                    pwrite_exact(self.fd, view, record.file_offset, self.sink.direct_io, self.tmp_path)
            finally:
                view.release()
        finally:
            self.free.put(buffer)
        return PageReadMetrics(read_seconds=time.perf_counter() - started,
                               logical_bytes=page.valid_tokens * self.layout.bytes_per_token,
                               physical_bytes=record.storage_bytes)

    def _release(self) -> None:
        self.memory_plan.release("bounce", self.registered_bytes)
        for b in self.buffers:
            b.close()
        self.closed = True

    def close(self) -> Path:
        if self.closed:
            return self.path
        try:
            try:
                try:
                    os.fsync(self.fd)
                finally:
                    os.close(self.fd)
                if self.tmp_path.stat().st_size != expected_file_size(self.pages):
                    raise OSError(errno.EIO, "output file size does not match its page table")
                os.replace(self.tmp_path, self.final_path)
                fsync_directory(self.path)
                atomic_write_json(self.path / "manifest.json", {
                    "format": "seqattn-output",
                    "version": FORMAT_VERSION,
                    "alignment_bytes": DIRECT_IO_ALIGNMENT,
                    "layout": self.layout.as_dict(),
                    "cu_seqlens": list(self.cu_seqlens),
                    "pages": [p.as_dict() for p in self.pages],
                    "files": {"output": {"name": "out.bin", "size_bytes": expected_file_size(self.pages)}},
                })
            except BaseException:
                for path in (self.tmp_path, self.final_path, self.path / "manifest.json.tmp"):
                    path.unlink(missing_ok=True)
                raise
        finally:
            self._release()
        return self.path

    def abort(self) -> None:
        if self.closed:
            return
        try:
            os.close(self.fd)
        finally:
            self._release()
        for path in (self.tmp_path, self.path / "manifest.json.tmp"):
            path.unlink(missing_ok=True)


class NvmeOutputSink(PageSink):
    backing_kind = "nvme"

    def __init__(self, path: str | os.PathLike[str], *, direct_io: bool = True) -> None:
        self.path = Path(path)
        self.direct_io = direct_io

    def open_writer(self, layout: TensorLayout, cu_seqlens: Sequence[int], pages: Sequence[PageDescriptor],
                    memory_plan: HostMemoryPlan, queue_depth: int) -> PageWriter:
        return _NvmeOutputWriter(self, layout, cu_seqlens, pages, memory_plan, queue_depth)


def load_nvme_output(path: str | os.PathLike[str], *, direct_io: bool = False) -> torch.Tensor:
    directory = Path(path)
    try:
        manifest = json.loads((directory / "manifest.json").read_text())
    except (OSError, json.JSONDecodeError) as error:
        raise ValueError("cannot read output manifest") from error
    if manifest.get("format") != "seqattn-output" or manifest.get("version") != FORMAT_VERSION:
        raise ValueError("unsupported or corrupt seqattn output manifest")
    layout = TensorLayout(**manifest["layout"])
    pages = tuple(PageDescriptor.from_dict(p) for p in manifest["pages"])
    output = torch.empty((layout.total_tokens, layout.heads, layout.head_dim), dtype=layout.torch_dtype)
    file_path = directory / manifest["files"]["output"]["name"]
    expected = int(manifest["files"]["output"]["size_bytes"])
    if file_path.stat().st_size != expected or expected_file_size(pages) != expected:
        raise ValueError("output file size does not match manifest")
    fd = open_file(file_path, os.O_RDONLY, 0, direct_io)
    buffer = AlignedBuffer(max((p.storage_bytes for p in pages), default=DIRECT_IO_ALIGNMENT))
    try:
        for page in pages:
            view = buffer.view(page.storage_bytes)
            try:
                pread_exact(fd, view, page.file_offset, direct_io, file_path)
            finally:
                view.release()
            target = output[page.token_start : page.token_stop]
            buffer.copy_to_tensor(0, target, target.numel())
    finally:
        os.close(fd)
        buffer.close()
    return output


@contextmanager
def ephemeral_nvme_directory(parent: str | os.PathLike[str] | None = None, *,
                             prefix: str = "seqattn-") -> Iterator[Path]:
    """Temporary store directory removed on exit."""
    path = Path(tempfile.mkdtemp(prefix=prefix, dir=parent))
    try:
        yield path
    finally:
        shutil.rmtree(path, ignore_errors=True)


__all__ = ["NvmeOutputSink", "ephemeral_nvme_directory", "load_nvme_output"]
