"""Builder of the aligned Q/K/V page store.

Produces the reference's format (src/seqattn_core/storage/qkv_writer.py:26-265
and storage/records.py): ``q.bin`` and ``kv.bin`` with one 4,096-byte aligned,
zero-padded record per page, and ``manifest.json`` with the same keys.  The
construction and error messages are the reference's; the write path is this
package's own:

* Every record is described as a list of (offset, bytes) pieces.  Buffered
  files write the pieces straight from the caller's page tensors, with the
  gaps and the tail filled from one shared zero block, as a single
  ``pwritev``; O_DIRECT files stage the record in an aligned page buffer
  first (O_DIRECT needs aligned source memory).
* Data goes to ``*.tmp`` files that are renamed into place, and the manifest
  is published last, so a build that fails or is interrupted never leaves a
  store that opens.
* INT8 K/V storage quantizes each page while it is written.
"""

from __future__ import annotations

import errno
import math
import os
import time
from collections.abc import Iterable, Iterator, Sequence
from pathlib import Path

import torch

from ..paged.layout import KVLayout, PageDescriptor, TensorLayout, build_page_descriptors
from ..paged.memory import MemoryPageSource
from ..quantization import quantize_int8_per_token_group
from .direct_io import DIRECT_IO_ALIGNMENT, FORMAT_VERSION, PageBuffer, RecordFile, byte_view, publish_json, sync_directory
from .qkv_store import NvmeQKVStore
from .records import expected_file_size, kv_record_pages, q_record_pages


class _RecordSink:
    """Writes records given as (offset within the record, CPU tensor) pieces."""

    def __init__(self, path: Path, largest_record: int, direct_io: bool) -> None:
        self.file = RecordFile(path, write=True, direct_io=direct_io)
        self.stage = PageBuffer(largest_record) if direct_io else None
        self.zeros = None if direct_io else bytes(largest_record)

    def write(self, page: PageDescriptor, pieces: Sequence[tuple[int, torch.Tensor]]) -> None:
        size = page.storage_bytes
        if self.stage is not None:
            self.stage.bytes[:size].zero_()
            for offset, tensor in pieces:
                self.stage.put(offset, tensor)
            window = self.stage.window(size)
            try:
                self.file.write_from(page.file_offset, window)
            finally:
                window.release()
            return
        views, cursor = [], 0
        for offset, tensor in sorted(pieces, key=lambda piece: piece[0]):
            if offset > cursor:
                views.append(memoryview(self.zeros)[: offset - cursor])
            data = byte_view(tensor.contiguous())
            views.append(data)
            cursor = offset + len(data)
        if cursor < size:
            views.append(memoryview(self.zeros)[: size - cursor])
        self.file.write_from(page.file_offset, *views)

    def finish(self) -> None:
        self.file.close(sync=True)
        self.release()

    def release(self) -> None:
        self.file.close()
        if self.stage is not None:
            self.stage.release()
            self.stage = None


def _take(pages: Iterator, what: str):
    try:
        return next(pages)
    except StopIteration:
        raise ValueError(f"{what} iterator ended early") from None


def _expect_end(pages: Iterator, what: str) -> None:
    if next(pages, None) is not None:
        raise ValueError(f"{what} iterator yielded extra pages")


class NvmeQKVWriter:
    """Streaming builder for an aligned, manifest-described Q/K/V store."""

    def __init__(
        self,
        path: str | os.PathLike[str],
        *,
        q_layout: TensorLayout,
        kv_layout: KVLayout,
        cu_seqlens_q: Sequence[int],
        cu_seqlens_k: Sequence[int],
        page_target_bytes: int = 16 * 2**20,
        block_n: int = 64,
        direct_io: bool = True,
    ) -> None:
        self.path = Path(path)
        self.q_layout = q_layout
        self.kv_layout = kv_layout
        self.cu_seqlens_q = tuple(int(x) for x in cu_seqlens_q)
        self.cu_seqlens_k = tuple(int(x) for x in cu_seqlens_k)
        self.page_target_bytes = page_target_bytes
        self.block_n = block_n
        self.direct_io = direct_io
        self.quantization_seconds = 0.0
        self.path.mkdir(parents=True, exist_ok=True)
        if (self.path / "manifest.json").exists():
            raise FileExistsError(f"store already exists: {self.path}")
        paging = {"page_target_bytes": page_target_bytes, "token_alignment": block_n}
        self.q_pages = q_record_pages(
            build_page_descriptors(self.cu_seqlens_q, bytes_per_token=q_layout.bytes_per_token, **paging), q_layout)
        self.kv_pages = kv_record_pages(
            build_page_descriptors(self.cu_seqlens_k, bytes_per_token=kv_layout.storage_bytes_per_token, **paging),
            kv_layout)
        self._staged = {"q": self.path / "q.bin.tmp", "kv": self.path / "kv.bin.tmp"}
        self._published = {"q": self.path / "q.bin", "kv": self.path / "kv.bin"}

    # -- page checks (the reference's messages) -----------------------------
    def _q_pieces(self, page: PageDescriptor, rows: torch.Tensor) -> list[tuple[int, torch.Tensor]]:
        shape = (page.valid_tokens, self.q_layout.heads, self.q_layout.head_dim)
        if rows.device.type != "cpu" or tuple(rows.shape) != shape:
            raise ValueError(f"query page {page.page_id} must use CPU shape {shape}")
        if rows.dtype != self.q_layout.torch_dtype:
            raise ValueError("query page dtype does not match q_layout")
        return [(0, rows)]

    def _kv_pieces(self, page: PageDescriptor, k: torch.Tensor, v: torch.Tensor,
                   scratch: dict[str, torch.Tensor]) -> list[tuple[int, torch.Tensor]]:
        layout = self.kv_layout
        shape = (page.valid_tokens, layout.heads, layout.head_dim)
        if k.device.type != "cpu" or v.device.type != "cpu":
            raise ValueError("K/V writer pages must be CPU tensors")
        if tuple(k.shape) != shape or tuple(v.shape) != shape:
            raise ValueError(f"K/V page {page.page_id} must use shape {shape}")
        if k.dtype != layout.source_torch_dtype or v.dtype != k.dtype:
            raise ValueError("K/V page dtype does not match kv_layout")
        if layout.storage_dtype != "int8":
            return [(0, k), (page.v_offset, v)]
        n = page.valid_tokens
        groups = math.ceil(n / layout.quant_group_tokens)
        started = time.perf_counter()
        for name, source in (("k", k), ("v", v)):
            quantize_int8_per_token_group(source, scratch[name][:n], scratch[name + "_scale"][:groups],
                                          group_tokens=layout.quant_group_tokens)
        self.quantization_seconds += time.perf_counter() - started
        return [(0, scratch["k"][:n]), (page.v_offset, scratch["v"][:n]),
                (page.k_scale_offset, scratch["k_scale"][:groups]), (page.v_scale_offset, scratch["v_scale"][:groups])]

    def _int8_scratch(self) -> dict[str, torch.Tensor]:
        rows = max((p.padded_tokens for p in self.kv_pages), default=0)
        if self.kv_layout.storage_dtype != "int8" or rows == 0:
            return {}
        shape = (rows, self.kv_layout.heads, self.kv_layout.head_dim)
        groups = (math.ceil(rows / self.kv_layout.quant_group_tokens), self.kv_layout.heads)
        return {"k": torch.empty(shape, dtype=torch.int8), "v": torch.empty(shape, dtype=torch.int8),
                "k_scale": torch.empty(groups, dtype=torch.float16),
                "v_scale": torch.empty(groups, dtype=torch.float16)}

    def _manifest(self) -> dict[str, object]:
        return {
            "format": "seqattn-qkv",
            "version": FORMAT_VERSION,
            "alignment_bytes": DIRECT_IO_ALIGNMENT,
            "page_target_bytes": self.page_target_bytes,
            "block_n": self.block_n,
            "q_layout": self.q_layout.as_dict(),
            "kv_layout": self.kv_layout.as_dict(),
            "cu_seqlens_q": list(self.cu_seqlens_q),
            "cu_seqlens_k": list(self.cu_seqlens_k),
            "q_pages": [p.as_dict() for p in self.q_pages],
            "kv_pages": [p.as_dict() for p in self.kv_pages],
            "files": {
                "q": {"name": "q.bin", "size_bytes": expected_file_size(self.q_pages)},
                "kv": {"name": "kv.bin", "size_bytes": expected_file_size(self.kv_pages)},
            },
            "quantization_seconds": self.quantization_seconds,
        }

    def write_pages(
        self,
        q_pages: Iterable[torch.Tensor],
        kv_pages: Iterable[tuple[torch.Tensor, torch.Tensor]],
    ) -> NvmeQKVStore:
        sinks: list[_RecordSink] = []
        try:
            largest = lambda pages: max((p.storage_bytes for p in pages), default=DIRECT_IO_ALIGNMENT)  # noqa: E731
            q_sink = _RecordSink(self._staged["q"], largest(self.q_pages), self.direct_io)
            sinks.append(q_sink)
            kv_sink = _RecordSink(self._staged["kv"], largest(self.kv_pages), self.direct_io)
            sinks.append(kv_sink)
            q_iter = iter(q_pages)
            for page in self.q_pages:
                q_sink.write(page, self._q_pieces(page, _take(q_iter, "query page")))
            _expect_end(q_iter, "query page")
            kv_iter = iter(kv_pages)
            scratch = self._int8_scratch()
            for page in self.kv_pages:
                k, v = _take(kv_iter, "K/V page")
                kv_sink.write(page, self._kv_pieces(page, k, v, scratch))
            _expect_end(kv_iter, "K/V page")
            for sink in sinks:
                sink.finish()
            sinks = []
            for key, pages, what in (("q", self.q_pages, "query"), ("kv", self.kv_pages, "K/V")):
                if self._staged[key].stat().st_size != expected_file_size(pages):
                    raise OSError(errno.EIO, f"{what} file size does not match its page table")
            for key in ("q", "kv"):
                os.replace(self._staged[key], self._published[key])
            sync_directory(self.path)
            publish_json(self.path / "manifest.json", self._manifest())
        except BaseException:
            for sink in sinks:
                sink.release()
            self.abort()
            raise
        return NvmeQKVStore(self.path, direct_io=self.direct_io)

    def abort(self) -> None:
        """Remove everything an unfinished build wrote (a published store,
        one with a manifest, is left alone)."""
        leftovers = [*self._staged.values(), self.path / "manifest.json.tmp"]
        if not (self.path / "manifest.json").exists():
            leftovers += list(self._published.values())
        for path in leftovers:
            path.unlink(missing_ok=True)

    @classmethod
    def from_tensors(
        cls,
        path: str | os.PathLike[str],
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        *,
        page_target_bytes: int = 16 * 2**20,
        block_n: int = 64,
        kv_storage_dtype: str | None = None,
        quant_group_tokens: int = 64,
        direct_io: bool = True,
    ) -> NvmeQKVStore:
        # The in-memory source validates the tensors and derives the layouts.
        source = MemoryPageSource(
            q=q, k=k, v=v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
            page_target_bytes=page_target_bytes, block_n=block_n,
            kv_storage_dtype=kv_storage_dtype, quant_group_tokens=quant_group_tokens,
        )
        writer = cls(
            path, q_layout=source.q_layout, kv_layout=source.kv_layout,
            cu_seqlens_q=source.cu_seqlens_q or (), cu_seqlens_k=source.cu_seqlens_k or (),
            page_target_bytes=page_target_bytes, block_n=block_n, direct_io=direct_io,
        )
        return writer.write_pages(
            (q[p.token_start : p.token_stop] for p in writer.q_pages),
            ((k[p.token_start : p.token_stop], v[p.token_start : p.token_stop]) for p in writer.kv_pages),
        )


__all__ = ["NvmeQKVWriter"]
