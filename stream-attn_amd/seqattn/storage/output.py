"""Aligned output page store.

Format, manifest keys and messages follow the reference
(src/seqattn_core/storage/output.py:31-251): one 4,096-byte aligned,
zero-padded record per query page in ``out.bin`` and a ``seqattn-output``
manifest published last.  The writer is this package's own: it shares the
record writer of the Q/K/V store builder (pieces written straight from the
page tensor for buffered files, staged in an aligned page buffer for
O_DIRECT), one per concurrent writer thread, so pages can be written in any
order from several I/O threads.
"""

from __future__ import annotations

import errno
import json
import os
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
from .direct_io import DIRECT_IO_ALIGNMENT, FORMAT_VERSION, BufferPool, RecordFile, byte_view, publish_json, sync_directory
from .records import expected_file_size, q_record_pages


class _OutputWriter(PageWriter):
    def __init__(self, sink: NvmeOutputSink, layout: TensorLayout, cu_seqlens: Sequence[int],
                 pages: Sequence[PageDescriptor], memory_plan: HostMemoryPlan, queue_depth: int) -> None:
        self.layout = layout
        self.cu_seqlens = tuple(cu_seqlens)
        self.pages = q_record_pages(pages, layout)
        self.by_id = {p.page_id: p for p in self.pages}
        self.directory = sink.path
        self.directory.mkdir(parents=True, exist_ok=True)
        if (self.directory / "manifest.json").exists():
            raise FileExistsError(f"output store already exists: {self.directory}")
        self.staged = self.directory / "out.bin.tmp"
        self.published = self.directory / "out.bin"
        largest = max((p.storage_bytes for p in self.pages), default=DIRECT_IO_ALIGNMENT)
        self.direct_io = sink.direct_io
        # O_DIRECT needs aligned staging memory, charged as bounce buffers;
        # buffered writes go straight from the page tensors.
        self.pool = BufferPool(queue_depth, largest, memory_plan) if self.direct_io else None
        self.zeros = None if self.direct_io else bytes(largest)
        try:
            self.file = RecordFile(self.staged, write=True, direct_io=self.direct_io)
        except BaseException:
            if self.pool is not None:
                self.pool.close()
            raise
        self.finished = False
        self._guard = threading.Lock()

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        record = self.by_id[page.page_id]
        rows = data[: page.valid_tokens]
        if data.device.type != "cpu" or tuple(rows.shape) != (page.valid_tokens, self.layout.heads,
                                                             self.layout.head_dim):
            raise ValueError("output page tensor does not match its descriptor")
        if data.dtype != self.layout.torch_dtype:
            raise ValueError("output page dtype does not match output layout")
        started = time.perf_counter()
        if self.pool is not None:
            with self.pool.lease() as buffer:
                buffer.bytes[: record.storage_bytes].zero_()
                buffer.put(0, rows)
                window = buffer.window(record.storage_bytes)
                try:
                    with self._guard:
                        self.file.write_from(record.file_offset, window)
                finally:
                    window.release()
        else:
            payload = byte_view(rows.contiguous())
            tail = memoryview(self.zeros)[: record.storage_bytes - len(payload)]
            with self._guard:
                self.file.write_from(record.file_offset, payload, tail)
        return PageReadMetrics(read_seconds=time.perf_counter() - started,
                               logical_bytes=page.valid_tokens * self.layout.bytes_per_token,
                               physical_bytes=record.storage_bytes)

    def _finish(self) -> None:
        self.file.close()
        if self.pool is not None:
            self.pool.close()
        self.finished = True

    def close(self) -> Path:
        if self.finished:
            return self.directory
        try:
            self.file.close(sync=True)
            if self.staged.stat().st_size != expected_file_size(self.pages):
                raise OSError(errno.EIO, "output file size does not match its page table")
            os.replace(self.staged, self.published)
            sync_directory(self.directory)
            publish_json(self.directory / "manifest.json", {
                "format": "seqattn-output",
                "version": FORMAT_VERSION,
                "alignment_bytes": DIRECT_IO_ALIGNMENT,
                "layout": self.layout.as_dict(),
                "cu_seqlens": list(self.cu_seqlens),
                "pages": [p.as_dict() for p in self.pages],
                "files": {"output": {"name": "out.bin", "size_bytes": expected_file_size(self.pages)}},
            })
        except BaseException:
            for path in (self.staged, self.published, self.directory / "manifest.json.tmp"):
                path.unlink(missing_ok=True)
            raise
        finally:
            self._finish()
        return self.directory

    def abort(self) -> None:
        if self.finished:
            return
        self._finish()
        for path in (self.staged, self.directory / "manifest.json.tmp"):
            path.unlink(missing_ok=True)


class NvmeOutputSink(PageSink):
    backing_kind = "nvme"

    def __init__(self, path: str | os.PathLike[str], *, direct_io: bool = True) -> None:
        self.path = Path(path)
        self.direct_io = direct_io

    def open_writer(self, layout: TensorLayout, cu_seqlens: Sequence[int], pages: Sequence[PageDescriptor],
                    memory_plan: HostMemoryPlan, queue_depth: int) -> PageWriter:
        return _OutputWriter(self, layout, cu_seqlens, pages, memory_plan, queue_depth)


def load_nvme_output(path: str | os.PathLike[str], *, direct_io: bool = False) -> torch.Tensor:
    """A finished output store as one ``[tokens, heads, head_dim]`` tensor."""
    directory = Path(path)
    try:
        manifest = json.loads((directory / "manifest.json").read_text())
    except (OSError, json.JSONDecodeError) as error:
        raise ValueError("cannot read output manifest") from error
    if manifest.get("format") != "seqattn-output" or manifest.get("version") != FORMAT_VERSION:
        raise ValueError("unsupported or corrupt seqattn output manifest")
    layout = TensorLayout(**manifest["layout"])
    pages = tuple(PageDescriptor.from_dict(p) for p in manifest["pages"])
    data_path = directory / manifest["files"]["output"]["name"]
    size = int(manifest["files"]["output"]["size_bytes"])
    if data_path.stat().st_size != size or expected_file_size(pages) != size:
        raise ValueError("output file size does not match manifest")
    output = torch.empty((layout.total_tokens, layout.heads, layout.head_dim), dtype=layout.torch_dtype)
    file = RecordFile(data_path, write=False, direct_io=direct_io)
    try:
        if not direct_io:
            for page in pages:
                file.read_into(page.file_offset, byte_view(output[page.token_start : page.token_stop]))
            return output
        pool = BufferPool(1, max((p.storage_bytes for p in pages), default=DIRECT_IO_ALIGNMENT))
        try:
            with pool.lease() as buffer:
                for page in pages:
                    window = buffer.window(page.storage_bytes)
                    try:
                        file.read_into(page.file_offset, window)
                    finally:
                        window.release()
                    rows = output[page.token_start : page.token_stop]
                    buffer.get(0, rows, rows.numel())
        finally:
            pool.close()
    finally:
        file.close()
    return output


@contextmanager
def ephemeral_nvme_directory(parent: str | os.PathLike[str] | None = None, *,
                             prefix: str = "seqattn-") -> Iterator[Path]:
    """A temporary store directory, removed with its contents on exit."""
    path = Path(tempfile.mkdtemp(prefix=prefix, dir=parent))
    try:
        yield path
    finally:
        shutil.rmtree(path, ignore_errors=True)


__all__ = ["NvmeOutputSink", "ephemeral_nvme_directory", "load_nvme_output"]
