"""Streaming builder of an aligned Q/K/V page store
(reference src/seqattn_core/storage/qkv_writer.py:26-262).

Pages are written whole (zero padded to their record size) into temporary
files that are renamed into place and described by a JSON manifest written
last, atomically; a failed or interrupted build leaves no manifest, so a
half-written store never opens.  INT8 K/V storage quantizes each page at
write time.
"""

from __future__ import annotations

import errno
import math
import os
import time
from collections.abc import Iterable, Sequence
from pathlib import Path

import torch

from ..paged.layout import KVLayout, PageDescriptor, TensorLayout, build_page_descriptors
from ..paged.memory import MemoryPageSource
from ..quantization import quantize_int8_per_token_group
from .direct_io import DIRECT_IO_ALIGNMENT, FORMAT_VERSION, AlignedFileWriter, atomic_write_json, fsync_directory
from .qkv_store import NvmeQKVStore
from .records import expected_file_size, kv_record_pages, q_record_pages


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
        self.q_tmp = self.path / "q.bin.tmp"
        self.kv_tmp = self.path / "kv.bin.tmp"
        self._temporary_paths = [self.q_tmp, self.kv_tmp, self.path / "manifest.json.tmp"]
        self.q_pages = q_record_pages(
            build_page_descriptors(self.cu_seqlens_q, bytes_per_token=q_layout.bytes_per_token,
                                   page_target_bytes=page_target_bytes, token_alignment=block_n),
            q_layout,
        )
        self.kv_pages = kv_record_pages(
            build_page_descriptors(self.cu_seqlens_k, bytes_per_token=kv_layout.storage_bytes_per_token,
                                   page_target_bytes=page_target_bytes, token_alignment=block_n),
            kv_layout,
        )

    def _check_q(self, page: PageDescriptor, tensor: torch.Tensor) -> None:
        expected = (page.valid_tokens, self.q_layout.heads, self.q_layout.head_dim)
        if tensor.device.type != "cpu" or tuple(tensor.shape) != expected:
            raise ValueError(f"query page {page.page_id} must use CPU shape {expected}")
        if tensor.dtype != self.q_layout.torch_dtype:
            raise ValueError("query page dtype does not match q_layout")

    def _check_kv(self, page: PageDescriptor, k: torch.Tensor, v: torch.Tensor) -> None:
        expected = (page.valid_tokens, self.kv_layout.heads, self.kv_layout.head_dim)
        if k.device.type != "cpu" or v.device.type != "cpu":
            raise ValueError("K/V writer pages must be CPU tensors")
        if tuple(k.shape) != expected or tuple(v.shape) != expected:
            raise ValueError(f"K/V page {page.page_id} must use shape {expected}")
        if k.dtype != self.kv_layout.source_torch_dtype or v.dtype != k.dtype:
            raise ValueError("K/V page dtype does not match kv_layout")

    @staticmethod
    def _exhausted(iterator, what: str) -> None:
        try:
            next(iterator)
        except StopIteration:
            return
        raise ValueError(f"{what} iterator yielded extra pages")

    def write_pages(
        self,
        q_pages: Iterable[torch.Tensor],
        kv_pages: Iterable[tuple[torch.Tensor, torch.Tensor]],
    ) -> NvmeQKVStore:
        q_iter, kv_iter = iter(q_pages), iter(kv_pages)
        q_file = kv_file = None
        try:
            q_file = AlignedFileWriter(
                self.q_tmp, max((p.storage_bytes for p in self.q_pages), default=DIRECT_IO_ALIGNMENT),
                self.direct_io)
            kv_file = AlignedFileWriter(
                self.kv_tmp, max((p.storage_bytes for p in self.kv_pages), default=DIRECT_IO_ALIGNMENT),
                self.direct_io)
            for page in self.q_pages:
                tensor = next(q_iter, None)
                if tensor is None:
                    raise ValueError("query page iterator ended early")
                self._check_q(page, tensor)
                q_file.buffer.zero(page.storage_bytes)
                q_file.buffer.copy_tensor(0, tensor)
                q_file.write(page.file_offset, page.storage_bytes)
            self._exhausted(q_iter, "query page")

            int8 = self.kv_layout.storage_dtype == "int8"
            most = max((p.padded_tokens for p in self.kv_pages), default=0)
            if int8 and most:
                shape = (most, self.kv_layout.heads, self.kv_layout.head_dim)
                kq, vq = torch.empty(shape, dtype=torch.int8), torch.empty(shape, dtype=torch.int8)
                groups_max = math.ceil(most / self.kv_layout.quant_group_tokens)
                ks = torch.empty((groups_max, self.kv_layout.heads), dtype=torch.float16)
                vs = torch.empty_like(ks)
            for page in self.kv_pages:
                pair = next(kv_iter, None)
                if pair is None:
                    raise ValueError("K/V page iterator ended early")
                k, v = pair
                self._check_kv(page, k, v)
                kv_file.buffer.zero(page.storage_bytes)
                if int8:
                    n = page.valid_tokens
                    groups = math.ceil(n / self.kv_layout.quant_group_tokens)
                    started = time.perf_counter()
                    quantize_int8_per_token_group(k, kq[:n], ks[:groups],
                                                  group_tokens=self.kv_layout.quant_group_tokens)
                    quantize_int8_per_token_group(v, vq[:n], vs[:groups],
                                                  group_tokens=self.kv_layout.quant_group_tokens)
                    self.quantization_seconds += time.perf_counter() - started
                    kv_file.buffer.copy_tensor(0, kq[:n])
                    kv_file.buffer.copy_tensor(page.v_offset, vq[:n])
                    kv_file.buffer.copy_tensor(page.k_scale_offset, ks[:groups])
                    kv_file.buffer.copy_tensor(page.v_scale_offset, vs[:groups])
                else:
                    kv_file.buffer.copy_tensor(0, k)
                    kv_file.buffer.copy_tensor(page.v_offset, v)
                kv_file.write(page.file_offset, page.storage_bytes)
            self._exhausted(kv_iter, "K/V page")

            q_file.close()
            kv_file.close()
            q_file = kv_file = None
            if self.q_tmp.stat().st_size != expected_file_size(self.q_pages):
                raise OSError(errno.EIO, "query file size does not match its page table")
            if self.kv_tmp.stat().st_size != expected_file_size(self.kv_pages):
                raise OSError(errno.EIO, "K/V file size does not match its page table")
            os.replace(self.q_tmp, self.path / "q.bin")
            os.replace(self.kv_tmp, self.path / "kv.bin")
            fsync_directory(self.path)
            atomic_write_json(self.path / "manifest.json", {
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
            })
            return NvmeQKVStore(self.path, direct_io=self.direct_io)
        except BaseException:
            for f in (q_file, kv_file):
                if f is not None:
                    f.close()
            self.abort()
            raise

    def abort(self) -> None:
        paths = list(self._temporary_paths)
        if not (self.path / "manifest.json").exists():
            paths += [self.path / "q.bin", self.path / "kv.bin"]
        for path in paths:
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
        layout_source = MemoryPageSource(
            q=q, k=k, v=v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
            page_target_bytes=page_target_bytes, block_n=block_n,
            kv_storage_dtype=kv_storage_dtype, quant_group_tokens=quant_group_tokens,
        )
        writer = cls(
            path, q_layout=layout_source.q_layout, kv_layout=layout_source.kv_layout,
            cu_seqlens_q=layout_source.cu_seqlens_q or (), cu_seqlens_k=layout_source.cu_seqlens_k or (),
            page_target_bytes=page_target_bytes, block_n=block_n, direct_io=direct_io,
        )
        return writer.write_pages(
            (q[p.token_start : p.token_stop] for p in writer.q_pages),
            ((k[p.token_start : p.token_stop], v[p.token_start : p.token_stop]) for p in writer.kv_pages),
        )


__all__ = ["NvmeQKVWriter"]
