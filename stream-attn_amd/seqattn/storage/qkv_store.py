"""Manifest-described, 4,096-byte aligned Q/K/V page store
(reference src/seqattn_core/storage/qkv_store.py:29-227; same manifest and
validation rules, so stores written by either implementation load here).

Besides the protocol's ``read_q`` / ``read_kv`` (through aligned bounce
buffers registered as ``bounce`` host memory), the reader offers
``read_kv_record``: one read of a whole K/V record into a caller buffer (the
paged runtime's page-locked slots), with no per-tensor unpacking.
"""

from __future__ import annotations

import json
import math
import os
import queue
import time
from collections.abc import Sequence
from pathlib import Path

import torch

from ..paged.layout import KVLayout, PageDescriptor, PageReadMetrics, TensorLayout, pages_by_segment
from ..paged.memory_budget import HostMemoryPlan
from ..paged.protocols import PageReader, PageSource
from .direct_io import DIRECT_IO_ALIGNMENT, FORMAT_VERSION, AlignedBuffer, open_file, pread_exact
from .records import expected_file_size


class _NvmePageReader(PageReader):
    def __init__(self, store: NvmeQKVStore, memory_plan: HostMemoryPlan, queue_depth: int) -> None:
        self.store = store
        self.direct_io = store.direct_io
        largest = max([p.storage_bytes for p in (*store.q_pages, *store.kv_pages)] or [DIRECT_IO_ALIGNMENT])
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
        self.q_fd = self.kv_fd = -1
        try:
            self.q_fd = open_file(store.q_path, os.O_RDONLY, 0, self.direct_io)
            self.kv_fd = open_file(store.kv_path, os.O_RDONLY, 0, self.direct_io)
        except BaseException:
            if self.q_fd >= 0:
                os.close(self.q_fd)
            memory_plan.release("bounce", self.registered_bytes)
            for b in self.buffers:
                b.close()
            raise
        self.closed = False

    def _read_record(self, fd: int, path: Path, page: PageDescriptor) -> tuple[AlignedBuffer, float]:
        buffer = self.free.get()
        started = time.perf_counter()
        view = buffer.view(page.storage_bytes)
        try:
            pread_exact(fd, view, page.file_offset, self.direct_io, path)
        except BaseException:
            self.free.put(buffer)
            raise
        finally:
            view.release()
        return buffer, time.perf_counter() - started

    def read_q(self, page: PageDescriptor, out: torch.Tensor) -> PageReadMetrics:
        layout = self.store.q_layout
        buffer, elapsed = self._read_record(self.q_fd, self.store.q_path, page)
        try:
            buffer.copy_to_tensor(0, out, page.valid_tokens * layout.heads * layout.head_dim)
            if out.shape[0] > page.valid_tokens:
                out[page.valid_tokens :].zero_()
        finally:
            self.free.put(buffer)
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=page.valid_tokens * layout.bytes_per_token,
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
        buffer, elapsed = self._read_record(self.kv_fd, self.store.kv_path, page)
        try:
            elements = page.valid_tokens * layout.heads * layout.head_dim
            buffer.copy_to_tensor(0, k_out, elements)
            buffer.copy_to_tensor(page.v_offset, v_out, elements)
            logical = 2 * elements * k_out.element_size()
            if layout.storage_dtype == "int8":
                if k_scales_out is None or v_scales_out is None:
                    raise ValueError("INT8 K/V reads require scale buffers")
                scale_elements = math.ceil(page.valid_tokens / layout.quant_group_tokens) * layout.heads
                buffer.copy_to_tensor(page.k_scale_offset, k_scales_out, scale_elements)
                buffer.copy_to_tensor(page.v_scale_offset, v_scales_out, scale_elements)
                logical += 2 * scale_elements * 2
            if k_out.shape[0] > page.valid_tokens:
                k_out[page.valid_tokens :].zero_()
                v_out[page.valid_tokens :].zero_()
        finally:
            self.free.put(buffer)
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=logical, physical_bytes=page.storage_bytes)

    def read_kv_record(self, page: PageDescriptor, destination: torch.Tensor) -> PageReadMetrics:
        """Read the whole K/V record of ``page`` into the uint8 CPU tensor
        ``destination`` (at least ``page.storage_bytes`` long).

        Buffered stores read straight into it.  O_DIRECT stores read into an
        aligned bounce buffer and copy: the kernel cannot map GPU-registered
        page-locked memory for a direct transfer (the read fails with EFAULT).
        """
        if self.direct_io:
            buffer, elapsed = self._read_record(self.kv_fd, self.store.kv_path, page)
            try:
                destination[: page.storage_bytes].copy_(buffer.bytes[: page.storage_bytes])
            finally:
                self.free.put(buffer)
        else:
            started = time.perf_counter()
            view = memoryview(destination.numpy())[: page.storage_bytes]
            try:
                pread_exact(self.kv_fd, view, page.file_offset, False, self.store.kv_path)
            finally:
                view.release()
            elapsed = time.perf_counter() - started
        logical = 2 * page.valid_tokens * self.store.kv_layout.storage_bytes_per_token
        if self.store.kv_layout.storage_dtype == "int8":
            groups = math.ceil(page.valid_tokens / self.store.kv_layout.quant_group_tokens)
            logical += 2 * groups * self.store.kv_layout.heads * 2
        return PageReadMetrics(read_seconds=elapsed, logical_bytes=logical, physical_bytes=page.storage_bytes)

    def close(self) -> None:
        if self.closed:
            return
        os.close(self.q_fd)
        os.close(self.kv_fd)
        self.memory_plan.release("bounce", self.registered_bytes)
        for b in self.buffers:
            b.close()
        self.closed = True


class NvmeQKVStore(PageSource):
    """Read side of a store written by ``NvmeQKVWriter``."""

    backing_kind = "nvme"

    def __init__(self, path: str | os.PathLike[str], *, direct_io: bool = True) -> None:
        self.path = Path(path)
        manifest_path = self.path / "manifest.json"
        try:
            manifest = json.loads(manifest_path.read_text())
        except (OSError, json.JSONDecodeError) as error:
            raise ValueError(f"cannot read valid store manifest: {manifest_path}") from error
        if manifest.get("format") != "seqattn-qkv" or manifest.get("version") != FORMAT_VERSION:
            raise ValueError("unsupported or corrupt seqattn Q/K/V manifest")
        if manifest.get("alignment_bytes") != DIRECT_IO_ALIGNMENT:
            raise ValueError("manifest alignment is incompatible with this runtime")
        try:
            self.q_layout = TensorLayout(**manifest["q_layout"])
            self.kv_layout = KVLayout(**manifest["kv_layout"])
            self.cu_seqlens_q = tuple(int(x) for x in manifest["cu_seqlens_q"])
            self.cu_seqlens_k = tuple(int(x) for x in manifest["cu_seqlens_k"])
            self.q_pages = tuple(PageDescriptor.from_dict(p) for p in manifest["q_pages"])
            self.kv_pages = tuple(PageDescriptor.from_dict(p) for p in manifest["kv_pages"])
            self.q_path = self.path / manifest["files"]["q"]["name"]
            self.kv_path = self.path / manifest["files"]["kv"]["name"]
            q_size = int(manifest["files"]["q"]["size_bytes"])
            kv_size = int(manifest["files"]["kv"]["size_bytes"])
        except (KeyError, TypeError, ValueError) as error:
            raise ValueError("manifest is missing required Q/K/V layout fields") from error
        self.direct_io = direct_io
        self.quantization_seconds = float(manifest.get("quantization_seconds", 0.0))
        self._validate_pages(self.q_pages, self.cu_seqlens_q, q_size, "q")
        self._validate_pages(self.kv_pages, self.cu_seqlens_k, kv_size, "kv")
        for data_path, expected in ((self.q_path, q_size), (self.kv_path, kv_size)):
            try:
                actual = data_path.stat().st_size
            except OSError as error:
                raise ValueError(f"manifest data file is missing: {data_path}") from error
            if actual != expected:
                raise ValueError(f"manifest size mismatch for {data_path.name}: {actual} != {expected}")

    @staticmethod
    def _validate_pages(pages: Sequence[PageDescriptor], cu_seqlens: Sequence[int], file_size: int,
                        name: str) -> None:
        next_id = 0
        for segment_id, group in enumerate(pages_by_segment(pages, len(cu_seqlens) - 1)):
            token = cu_seqlens[segment_id]
            for page in group:
                if page.page_id != next_id:
                    raise ValueError(f"{name} page ids are not contiguous")
                if page.token_start != token or page.segment_id != segment_id:
                    raise ValueError(f"{name} page table crosses or skips a segment boundary")
                if page.valid_tokens <= 0 or page.padded_tokens < page.valid_tokens:
                    raise ValueError(f"{name} page has invalid token counts")
                if page.file_offset % DIRECT_IO_ALIGNMENT or page.storage_bytes % DIRECT_IO_ALIGNMENT:
                    raise ValueError(f"{name} page is not direct-I/O aligned")
                if page.payload_bytes + page.padding_bytes != page.storage_bytes:
                    raise ValueError(f"{name} page padding metadata is inconsistent")
                token = page.token_stop
                next_id += 1
            if token != cu_seqlens[segment_id + 1]:
                raise ValueError(f"{name} pages do not cover segment {segment_id}")
        if expected_file_size(pages) != file_size:
            raise ValueError(f"{name} page table does not match file size")

    def open_reader(self, memory_plan: HostMemoryPlan, queue_depth: int) -> PageReader:
        return _NvmePageReader(self, memory_plan, queue_depth)


__all__ = ["NvmeQKVStore"]
