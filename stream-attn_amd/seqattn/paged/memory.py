"""In-memory page sources and sinks.

Same classes, constructors, validation messages and metrics as the
reference (src/seqattn_core/paged/memory.py:106-343): ``MemoryPageSource``
pages caller-owned CPU tensors (which do not count toward the operator's
host budget), ``MemoryPageSink`` writes output pages into a caller-owned CPU
tensor, ``CallbackOutputSink`` hands each output page to a callback.

The MI355X runtime prefers not to copy at all: when the caller's tensors are
page-locked and stored in their own dtype, the paged runner gathers K/V rows
for the GPU straight from them (``pinned_kv_rows`` / ``pinned_q_rows``) and a
``MemoryPageSink`` over a page-locked tensor receives its rows by D2H directly
(``pinned_rows``).  The reader/writer protocol below serves every other case.
"""

from __future__ import annotations

import math
import time
from collections.abc import Callable, Sequence

import torch

from ..quantization import quantize_int8_per_token_group
from .layout import (
    KVLayout,
    PageDescriptor,
    PageReadMetrics,
    TensorLayout,
    build_page_descriptors,
    dtype_name,
    torch_dtype,
    validate_cu_seqlens,
)
from .memory_budget import HostMemoryPlan
from .protocols import PageReader, PageSink, PageSource, PageWriter

_STORAGE_DTYPES = ("bf16", "fp16", "fp32", "int8")


def _nbytes(tensor: torch.Tensor) -> int:
    return tensor.numel() * tensor.element_size()


def _fill_rows(out: torch.Tensor, rows: torch.Tensor) -> None:
    """``out[:len(rows)] = rows`` and zeros in the rest of ``out``."""
    count = rows.shape[0]
    out[:count].copy_(rows)
    if out.shape[0] > count:
        out[count:].zero_()


def _timed(started: float, logical: int, quantization: float = 0.0) -> PageReadMetrics:
    return PageReadMetrics(read_seconds=time.perf_counter() - started, quantization_seconds=quantization,
                           logical_bytes=logical, physical_bytes=logical)


def _check_source_tensors(q, k, v) -> None:
    if q is None and k is None:
        raise ValueError("at least one of q or k/v must be supplied")
    if (k is None) != (v is None):
        raise ValueError("k and v must be supplied together")
    for name, tensor in (("q", q), ("k", k), ("v", v)):
        if tensor is None:
            continue
        if tensor.device.type != "cpu" or tensor.ndim != 3 or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous CPU [tokens, heads, head_dim]")
    if k is None:
        return
    if k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("k and v must have matching shape and dtype")
    if q is not None:
        if q.shape[2] != k.shape[2] or q.shape[1] % k.shape[1]:
            raise ValueError("q and k/v head shapes are incompatible")
        if q.dtype != k.dtype:
            raise ValueError("q and k/v source dtype must match")


class _TensorPageReader(PageReader):
    """Pages of a ``MemoryPageSource`` copied (or INT8-quantized) into the
    runtime's page buffers."""

    def __init__(self, source: MemoryPageSource) -> None:
        self.source = source

    def read_q(self, page: PageDescriptor, out: torch.Tensor) -> PageReadMetrics:
        q = self.source.q
        if q is None:
            raise ValueError("this MemoryPageSource has no query tensor")
        started = time.perf_counter()
        rows = q[page.token_start : page.token_stop]
        _fill_rows(out, rows)
        return _timed(started, _nbytes(rows))

    def read_kv(
        self,
        page: PageDescriptor,
        k_out: torch.Tensor,
        v_out: torch.Tensor,
        k_scales_out: torch.Tensor | None = None,
        v_scales_out: torch.Tensor | None = None,
    ) -> PageReadMetrics:
        src = self.source
        if src.k is None or src.v is None or src.kv_layout is None:
            raise ValueError("this MemoryPageSource has no K/V tensors")
        layout = src.kv_layout
        started = time.perf_counter()
        span = slice(page.token_start, page.token_stop)
        n = page.valid_tokens
        logical = 2 * n * layout.storage_bytes_per_token
        quantization = 0.0
        if layout.storage_dtype != "int8":
            _fill_rows(k_out, src.k[span])
            _fill_rows(v_out, src.v[span])
            return _timed(started, logical)
        if k_scales_out is None or v_scales_out is None:
            raise ValueError("INT8 K/V reads require scale buffers")
        groups = math.ceil(n / layout.quant_group_tokens)
        began = time.perf_counter()
        for rows, codes, scales in ((src.k[span], k_out, k_scales_out), (src.v[span], v_out, v_scales_out)):
            quantize_int8_per_token_group(rows, codes[:n], scales[:groups], group_tokens=layout.quant_group_tokens)
            if codes.shape[0] > n:
                codes[n:].zero_()
        quantization = time.perf_counter() - began
        return _timed(started, logical + 2 * groups * layout.heads * 2, quantization)


class MemoryPageSource(PageSource):
    """Page source over caller-owned CPU tensors.

    The complete tensors do not count toward the paged operator's host budget.
    """

    def __init__(
        self,
        *,
        q: torch.Tensor | None = None,
        k: torch.Tensor | None = None,
        v: torch.Tensor | None = None,
        cu_seqlens_q: torch.Tensor | None = None,
        cu_seqlens_k: torch.Tensor | None = None,
        page_target_bytes: int = 16 * 2**20,
        block_n: int = 64,
        kv_storage_dtype: str | None = None,
        quant_group_tokens: int = 64,
    ) -> None:
        _check_source_tensors(q, k, v)
        self.q, self.k, self.v = q, k, v
        self.q_layout: TensorLayout | None = None
        self.kv_layout: KVLayout | None = None
        self.q_pages: tuple[PageDescriptor, ...] = ()
        self.kv_pages: tuple[PageDescriptor, ...] = ()
        self.cu_seqlens_q: tuple[int, ...] | None = None
        self.cu_seqlens_k: tuple[int, ...] | None = None
        paging = {"page_target_bytes": page_target_bytes, "token_alignment": block_n}
        if q is not None:
            if cu_seqlens_q is None:
                raise ValueError("cu_seqlens_q is required with q")
            self.cu_seqlens_q = tuple(validate_cu_seqlens(cu_seqlens_q, q.shape[0], "cu_seqlens_q"))
            self.q_layout = TensorLayout(q.shape[0], q.shape[1], q.shape[2], dtype_name(q.dtype))
            self.q_pages = build_page_descriptors(self.cu_seqlens_q, bytes_per_token=self.q_layout.bytes_per_token,
                                                  **paging)
        if k is not None:
            if cu_seqlens_k is None:
                raise ValueError("cu_seqlens_k is required with k/v")
            self.cu_seqlens_k = tuple(validate_cu_seqlens(cu_seqlens_k, k.shape[0], "cu_seqlens_k"))
            source_dtype = dtype_name(k.dtype)
            storage = kv_storage_dtype or source_dtype
            if storage not in _STORAGE_DTYPES:
                raise ValueError("unsupported K/V storage dtype")
            if storage != "int8" and torch_dtype(storage) != k.dtype:
                raise ValueError("exact K/V storage dtype must match the source dtype")
            self.kv_layout = KVLayout(k.shape[0], k.shape[1], k.shape[2], source_dtype, storage, quant_group_tokens)
            self.kv_pages = build_page_descriptors(
                self.cu_seqlens_k, bytes_per_token=self.kv_layout.storage_bytes_per_token, **paging)

    def open_reader(self, memory_plan: HostMemoryPlan, queue_depth: int) -> PageReader:
        del memory_plan, queue_depth  # nothing to buffer: rows come from the caller's tensors
        return _TensorPageReader(self)

    def pinned_q_rows(self, start: int, stop: int) -> torch.Tensor | None:
        """Page-locked view of query rows [start, stop), or None."""
        if self.q is not None and self.q.is_pinned():
            return self.q[start:stop]
        return None

    def pinned_kv_rows(self, start: int, stop: int) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Page-locked views of K/V rows [start, stop) in storage dtype, or None."""
        layout = self.kv_layout
        exact = layout is not None and layout.storage_dtype == layout.source_dtype
        if exact and self.k.is_pinned() and self.v.is_pinned():
            return self.k[start:stop], self.v[start:stop]
        return None


class _TensorPageWriter(PageWriter):
    def __init__(self, out: torch.Tensor | None, layout: TensorLayout) -> None:
        if out is None:
            raise ValueError("MemoryPageSink requires a caller-owned output tensor")
        if tuple(out.shape) != (layout.total_tokens, layout.heads, layout.head_dim):
            raise ValueError("MemoryPageSink output shape does not match the query layout")
        if out.dtype != layout.torch_dtype or out.device.type != "cpu":
            raise ValueError("MemoryPageSink output must be a matching CPU tensor")
        self.out = out

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        started = time.perf_counter()
        rows = data[: page.valid_tokens]
        self.out[page.token_start : page.token_stop].copy_(rows)
        return _timed(started, _nbytes(rows))

    def pinned_rows(self, start: int, stop: int) -> torch.Tensor | None:
        """Page-locked view of output rows [start, stop) for direct D2H, or None."""
        if self.out.is_pinned() and self.out.is_contiguous():
            return self.out[start:stop]
        return None

    def close(self) -> torch.Tensor:
        return self.out


class MemoryPageSink(PageSink):
    """Writes output pages into a caller-owned complete CPU tensor."""

    def __init__(self, out: torch.Tensor) -> None:
        self.out = out

    def open_writer(
        self,
        layout: TensorLayout,
        cu_seqlens: Sequence[int],
        pages: Sequence[PageDescriptor],
        memory_plan: HostMemoryPlan,
        queue_depth: int,
    ) -> PageWriter:
        del cu_seqlens, pages, memory_plan, queue_depth
        return _TensorPageWriter(self.out, layout)


class _CallbackPageWriter(PageWriter):
    def __init__(self, callback: Callable[[PageDescriptor, torch.Tensor], object]) -> None:
        self.callback = callback
        self.pages_written = 0

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        started = time.perf_counter()
        rows = data[: page.valid_tokens]
        self.callback(page, rows)
        self.pages_written += 1
        return _timed(started, _nbytes(rows))

    def close(self) -> int:
        return self.pages_written


class CallbackOutputSink(PageSink):
    """Synchronously hands each output page to a caller callback."""

    def __init__(self, callback: Callable[[PageDescriptor, torch.Tensor], object]) -> None:
        self.callback = callback

    def open_writer(
        self,
        layout: TensorLayout,
        cu_seqlens: Sequence[int],
        pages: Sequence[PageDescriptor],
        memory_plan: HostMemoryPlan,
        queue_depth: int,
    ) -> PageWriter:
        del layout, cu_seqlens, pages, memory_plan, queue_depth
        return _CallbackPageWriter(self.callback)


__all__ = ["CallbackOutputSink", "MemoryPageSink", "MemoryPageSource"]
