"""Read side of the aligned Q/K/V page store.

Format and manifest follow the reference (src/seqattn_core/storage/
qkv_store.py:150-227 and storage/records.py), with the same validation rules
and messages, so a store written by either implementation opens in the
other.  The reader is this package's own:

* Buffered stores read rows straight from the file into the caller's
  tensors (one ``preadv`` per contiguous range: the Q rows, the K rows, the V
  rows, the INT8 scale rows), with no bounce copy and no bounce memory.
* O_DIRECT stores read whole aligned records into page buffers lent by a
  pool sized to the I/O queue depth and charged to the host-memory plan's
  ``bounce`` category, then copy the rows out.
* ``read_kv_record`` hands the paged runtime a whole K/V record at once (for
  its page-locked cache slots), which avoids unpacking it into tensors.
"""

from __future__ import annotations

import json
import math
import os
import time
from collections.abc import Sequence
from pathlib import Path

import torch

from ..paged.layout import KVLayout, PageDescriptor, PageReadMetrics, TensorLayout, pages_by_segment
from ..paged.memory_budget import HostMemoryPlan
from ..paged.protocols import PageReader, PageSource
from .direct_io import DIRECT_IO_ALIGNMENT, FORMAT_VERSION, BufferPool, RecordFile, byte_view
from .records import expected_file_size


def _rows(tensor: torch.Tensor, count: int) -> memoryview:
    """Bytes of the first ``count`` rows of a contiguous CPU tensor."""
    if not tensor.is_contiguous():
        raise ValueError("page buffers must be contiguous CPU tensors")
    return byte_view(tensor[:count])


def _clear_tail(tensor: torch.Tensor | None, valid: int) -> None:
    if tensor is not None and tensor.shape[0] > valid:
        tensor[valid:].zero_()


def _kv_logical_bytes(page: PageDescriptor, layout: KVLayout) -> int:
    total = 2 * page.valid_tokens * layout.storage_bytes_per_token
    if layout.storage_dtype == "int8":
        total += 2 * math.ceil(page.valid_tokens / layout.quant_group_tokens) * layout.heads * 2
    return total


class _StoreReader(PageReader):
    def __init__(self, store: NvmeQKVStore, memory_plan: HostMemoryPlan, queue_depth: int) -> None:
        self.store = store
        self.pool: BufferPool | None = None
        self.files: list[RecordFile] = []
        try:
            if store.direct_io:
                largest = max((p.storage_bytes for p in (*store.q_pages, *store.kv_pages)),
                              default=DIRECT_IO_ALIGNMENT)
                self.pool = BufferPool(queue_depth, largest, memory_plan)
            self.q_file = RecordFile(store.q_path, write=False, direct_io=store.direct_io)
            self.files.append(self.q_file)
            self.kv_file = RecordFile(store.kv_path, write=False, direct_io=store.direct_io)
            self.files.append(self.kv_file)
        except BaseException:
            self.close()
            raise

    # -- whole records through a page buffer (O_DIRECT) -------------------
    def _bounced(self, file: RecordFile, page: PageDescriptor, unpack) -> float:
        with self.pool.lease() as buffer:
            started = time.perf_counter()
            window = buffer.window(page.storage_bytes)
            try:
                file.read_into(page.file_offset, window)
            finally:
                window.release()
            elapsed = time.perf_counter() - started
            unpack(buffer)
        return elapsed

    def read_q(self, page: PageDescriptor, out: torch.Tensor) -> PageReadMetrics:
        layout = self.store.q_layout
        n = page.valid_tokens
        if self.pool is not None:
            elapsed = self._bounced(self.q_file, page,
                                    lambda buffer: buffer.get(0, out, n * layout.heads * layout.head_dim))
        else:
            started = time.perf_counter()
            self.q_file.read_into(page.file_offset, _rows(out, n))
            elapsed = time.perf_counter() - started
        _clear_tail(out, n)
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=n * layout.bytes_per_token,
                               physical_bytes=page.storage_bytes)

    def read_kv(
        self,
        page: PageDescriptor,
        k_out: torch.Tensor,
        v_out: torch.Tensor,
        k_scales_out: torch.Tensor | None = None,
        v_scales_out: torch.Tensor | None = None,
    ) -> PageReadMetrics:
        layout = self.store.kv_layout
        n = page.valid_tokens
        quantized = layout.storage_dtype == "int8"
        if quantized and (k_scales_out is None or v_scales_out is None):
            raise ValueError("INT8 K/V reads require scale buffers")
        groups = math.ceil(n / layout.quant_group_tokens) if quantized else 0
        # (record offset, destination, rows) of every range the caller receives.
        parts = [(0, k_out, n), (page.v_offset, v_out, n)]
        if quantized:
            parts += [(page.k_scale_offset, k_scales_out, groups), (page.v_scale_offset, v_scales_out, groups)]
        if self.pool is not None:
            def unpack(buffer):
                for offset, tensor, rows in parts:
                    buffer.get(offset, tensor, rows * math.prod(tensor.shape[1:]))

            elapsed = self._bounced(self.kv_file, page, unpack)
        else:
            started = time.perf_counter()
            for offset, tensor, rows in parts:
                self.kv_file.read_into(page.file_offset + offset, _rows(tensor, rows))
            elapsed = time.perf_counter() - started
        _clear_tail(k_out, n)
        _clear_tail(v_out, n)
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=_kv_logical_bytes(page, layout),
                               physical_bytes=page.storage_bytes)

    def read_kv_record(self, page: PageDescriptor, destination: torch.Tensor) -> PageReadMetrics:
        """Read the whole K/V record of ``page`` into the uint8 CPU tensor
        ``destination`` (at least ``page.storage_bytes`` long).

        Buffered stores read straight into it.  O_DIRECT stores read into a
        page buffer and copy: the kernel cannot map GPU-registered page-locked
        memory for a direct transfer (the read fails with EFAULT).
        """
        size = page.storage_bytes
        if self.pool is not None:
            elapsed = self._bounced(self.kv_file, page,
                                    lambda buffer: destination[:size].copy_(buffer.bytes[:size]))
        else:
            started = time.perf_counter()
            view = byte_view(destination[:size])
            try:
                self.kv_file.read_into(page.file_offset, view)
            finally:
                view.release()
            elapsed = time.perf_counter() - started
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=_kv_logical_bytes(page, self.store.kv_layout),
                               physical_bytes=size)

    def close(self) -> None:
        for file in self.files:
            file.close()
        self.files = []
        if self.pool is not None:
            self.pool.close()
            self.pool = None


def _load_manifest(path: Path) -> dict:
    manifest_path = path / "manifest.json"
    try:
        manifest = json.loads(manifest_path.read_text())
    except (OSError, json.JSONDecodeError) as error:
        raise ValueError(f"cannot read valid store manifest: {manifest_path}") from error
    if manifest.get("format") != "seqattn-qkv" or manifest.get("version") != FORMAT_VERSION:
        raise ValueError("unsupported or corrupt seqattn Q/K/V manifest")
    if manifest.get("alignment_bytes") != DIRECT_IO_ALIGNMENT:
        raise ValueError("manifest alignment is incompatible with this runtime")
    return manifest


def check_page_table(pages: Sequence[PageDescriptor], cu_seqlens: Sequence[int], file_size: int,
                     name: str) -> None:
    """A page table must tile every segment with contiguous, aligned records
    that end exactly at the file's size."""
    expected_id = 0
    for segment, members in enumerate(pages_by_segment(pages, len(cu_seqlens) - 1)):
        cursor = cu_seqlens[segment]
        for page in members:
            problems = (
                (page.page_id != expected_id, "page ids are not contiguous"),
                (page.token_start != cursor or page.segment_id != segment,
                 "page table crosses or skips a segment boundary"),
                (page.valid_tokens <= 0 or page.padded_tokens < page.valid_tokens, "page has invalid token counts"),
                (page.file_offset % DIRECT_IO_ALIGNMENT != 0 or page.storage_bytes % DIRECT_IO_ALIGNMENT != 0,
                 "page is not direct-I/O aligned"),
                (page.payload_bytes + page.padding_bytes != page.storage_bytes,
                 "page padding metadata is inconsistent"),
            )
            for failed, message in problems:
                if failed:
                    raise ValueError(f"{name} {message}")
            cursor = page.token_stop
            expected_id += 1
        if cursor != cu_seqlens[segment + 1]:
            raise ValueError(f"{name} pages do not cover segment {segment}")
    if expected_file_size(pages) != file_size:
        raise ValueError(f"{name} page table does not match file size")


class NvmeQKVStore(PageSource):
    """Read side of a store written by ``NvmeQKVWriter``."""

    backing_kind = "nvme"

    def __init__(self, path: str | os.PathLike[str], *, direct_io: bool = True) -> None:
        self.path = Path(path)
        self.direct_io = direct_io
        manifest = _load_manifest(self.path)
        try:
            files = manifest["files"]
            self.q_layout = TensorLayout(**manifest["q_layout"])
            self.kv_layout = KVLayout(**manifest["kv_layout"])
            self.cu_seqlens_q = tuple(int(x) for x in manifest["cu_seqlens_q"])
            self.cu_seqlens_k = tuple(int(x) for x in manifest["cu_seqlens_k"])
            self.q_pages = tuple(PageDescriptor.from_dict(p) for p in manifest["q_pages"])
            self.kv_pages = tuple(PageDescriptor.from_dict(p) for p in manifest["kv_pages"])
            self.q_path = self.path / files["q"]["name"]
            self.kv_path = self.path / files["kv"]["name"]
            sizes = {"q": int(files["q"]["size_bytes"]), "kv": int(files["kv"]["size_bytes"])}
        except (KeyError, TypeError, ValueError) as error:
            raise ValueError("manifest is missing required Q/K/V layout fields") from error
        self.quantization_seconds = float(manifest.get("quantization_seconds", 0.0))
        check_page_table(self.q_pages, self.cu_seqlens_q, sizes["q"], "q")
        check_page_table(self.kv_pages, self.cu_seqlens_k, sizes["kv"], "kv")
        for data_path, expected in ((self.q_path, sizes["q"]), (self.kv_path, sizes["kv"])):
            try:
                actual = data_path.stat().st_size
            except OSError as error:
                raise ValueError(f"manifest data file is missing: {data_path}") from error
            if actual != expected:
                raise ValueError(f"manifest size mismatch for {data_path.name}: {actual} != {expected}")

    def open_reader(self, memory_plan: HostMemoryPlan, queue_depth: int) -> PageReader:
        return _StoreReader(self, memory_plan, queue_depth)


__all__ = ["NvmeQKVStore", "check_page_table"]
