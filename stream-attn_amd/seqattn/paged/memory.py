"""In-memory page sources and sinks (reference src/seqattn_core/paged/memory.py:106-343).

``MemoryPageSource`` pages caller-owned CPU tensors (which do not count
toward the operator's host budget); ``MemoryPageSink`` writes output pages
into a caller-owned CPU tensor; ``CallbackOutputSink`` hands each output page
to a callback.  Same constructors, validation messages and metrics as the
reference.

Zero-copy: when the caller's tensors are page-locked and stored in their own
dtype, the paged runner gathers K/V pages straight from them
(``pinned_kv_rows``) and a ``MemoryPageSink`` over a page-locked tensor
receives its rows by D2H directly (``pinned_rows``); the reader/writer
protocol is used otherwise.
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


def _zero_tail(out: torch.Tensor, valid: int) -> None:
    if out.shape[0] > valid:
        out[valid:].zero_()


class _MemoryReader(PageReader):
    def __init__(self, source: MemoryPageSource) -> None:
        self.source = source

    def read_q(self, page: PageDescriptor, out: torch.Tensor) -> PageReadMetrics:
        if self.source.q is None:
            raise ValueError("this MemoryPageSource has no query tensor")
        started = time.perf_counter()
        rows = self.source.q[page.token_start : page.token_stop]
        out[: page.valid_tokens].copy_(rows)
        _zero_tail(out, page.valid_tokens)
        size = rows.numel() * rows.element_size()
        return PageReadMetrics(read_seconds=time.perf_counter() - started, logical_bytes=size, physical_bytes=size)

    def read_kv(
        self,
        page: PageDescriptor,
        k_out: torch.Tensor,
        v_out: torch.Tensor,
        k_scales_out: torch.Tensor | None = None,
        v_scales_out: torch.Tensor | None = None,
    ) -> PageReadMetrics:
        source = self.source
        if source.k is None or source.v is None or source.kv_layout is None:
            raise ValueError("this MemoryPageSource has no K/V tensors")
        layout = source.kv_layout
        started = time.perf_counter()
        k_rows = source.k[page.token_start : page.token_stop]
        v_rows = source.v[page.token_start : page.token_stop]
        n = page.valid_tokens
        quant_seconds = 0.0
        logical = 2 * n * layout.storage_bytes_per_token
        if layout.storage_dtype == "int8":
            if k_scales_out is None or v_scales_out is None:
                raise ValueError("INT8 K/V reads require scale buffers")
            groups = math.ceil(n / layout.quant_group_tokens)
            quant_started = time.perf_counter()
            quantize_int8_per_token_group(k_rows, k_out[:n], k_scales_out[:groups],
                                          group_tokens=layout.quant_group_tokens)
            quantize_int8_per_token_group(v_rows, v_out[:n], v_scales_out[:groups],
                                          group_tokens=layout.quant_group_tokens)
            quant_seconds = time.perf_counter() - quant_started
            logical += 2 * groups * layout.heads * 2
        else:
            k_out[:n].copy_(k_rows)
            v_out[:n].copy_(v_rows)
        _zero_tail(k_out, n)
        _zero_tail(v_out, n)
        return PageReadMetrics(
            read_seconds=time.perf_counter() - started,
            quantization_seconds=quant_seconds,
            logical_bytes=logical,
            physical_bytes=logical,
        )


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
        if q is None and k is None:
            raise ValueError("at least one of q or k/v must be supplied")
        if (k is None) != (v is None):
            raise ValueError("k and v must be supplied together")
        for name, tensor in (("q", q), ("k", k), ("v", v)):
            if tensor is not None and (
                tensor.device.type != "cpu" or tensor.ndim != 3 or not tensor.is_contiguous()
            ):
                raise ValueError(f"{name} must be contiguous CPU [tokens, heads, head_dim]")
        if k is not None and (k.shape != v.shape or k.dtype != v.dtype):
            raise ValueError("k and v must have matching shape and dtype")
        if q is not None and k is not None:
            if q.shape[2] != k.shape[2] or q.shape[1] % k.shape[1]:
                raise ValueError("q and k/v head shapes are incompatible")
            if q.dtype != k.dtype:
                raise ValueError("q and k/v source dtype must match")
        self.q, self.k, self.v = q, k, v
        self.q_layout: TensorLayout | None = None
        self.kv_layout: KVLayout | None = None
        self.q_pages: tuple[PageDescriptor, ...] = ()
        self.kv_pages: tuple[PageDescriptor, ...] = ()
        self.cu_seqlens_q: tuple[int, ...] | None = None
        self.cu_seqlens_k: tuple[int, ...] | None = None
        if q is not None:
            if cu_seqlens_q is None:
                raise ValueError("cu_seqlens_q is required with q")
            q_bounds = validate_cu_seqlens(cu_seqlens_q, q.shape[0], "cu_seqlens_q")
            self.cu_seqlens_q = tuple(q_bounds)
            self.q_layout = TensorLayout(q.shape[0], q.shape[1], q.shape[2], dtype_name(q.dtype))
            self.q_pages = build_page_descriptors(
                q_bounds, bytes_per_token=self.q_layout.bytes_per_token,
                page_target_bytes=page_target_bytes, token_alignment=block_n,
            )
        if k is not None:
            if cu_seqlens_k is None:
                raise ValueError("cu_seqlens_k is required with k/v")
            k_bounds = validate_cu_seqlens(cu_seqlens_k, k.shape[0], "cu_seqlens_k")
            self.cu_seqlens_k = tuple(k_bounds)
            storage = dtype_name(k.dtype) if kv_storage_dtype is None else kv_storage_dtype
            if storage not in {"bf16", "fp16", "fp32", "int8"}:
                raise ValueError("unsupported K/V storage dtype")
            if storage != "int8" and torch_dtype(storage) != k.dtype:
                raise ValueError("exact K/V storage dtype must match the source dtype")
            self.kv_layout = KVLayout(k.shape[0], k.shape[1], k.shape[2], dtype_name(k.dtype), storage,
                                      quant_group_tokens)
            self.kv_pages = build_page_descriptors(
                k_bounds, bytes_per_token=self.kv_layout.storage_bytes_per_token,
                page_target_bytes=page_target_bytes, token_alignment=block_n,
            )

    def open_reader(self, memory_plan: HostMemoryPlan, queue_depth: int) -> PageReader:
        del memory_plan, queue_depth
        return _MemoryReader(self)

    def pinned_q_rows(self, start: int, stop: int) -> torch.Tensor | None:
        """Page-locked view of query rows [start, stop), or None."""
        if self.q is None or not self.q.is_pinned():
            return None
        return self.q[start:stop]

    def pinned_kv_rows(self, start: int, stop: int) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Page-locked views of K/V rows [start, stop) in storage dtype, or None."""
        if (
            self.k is None
            or self.kv_layout is None
            or self.kv_layout.storage_dtype != self.kv_layout.source_dtype
            or not (self.k.is_pinned() and self.v.is_pinned())
        ):
            return None
        return self.k[start:stop], self.v[start:stop]


class _MemoryPageWriter(PageWriter):
    def __init__(self, sink: MemoryPageSink, layout: TensorLayout) -> None:
        self.sink = sink
        out = sink.out
        if out is None:
            raise ValueError("MemoryPageSink requires a caller-owned output tensor")
        if tuple(out.shape) != (layout.total_tokens, layout.heads, layout.head_dim):
            raise ValueError("MemoryPageSink output shape does not match the query layout")
        if out.dtype != layout.torch_dtype or out.device.type != "cpu":
            raise ValueError("MemoryPageSink output must be a matching CPU tensor")

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        started = time.perf_counter()
        self.sink.out[page.token_start : page.token_stop].copy_(data[: page.valid_tokens])
        size = page.valid_tokens * data.shape[1] * data.shape[2] * data.element_size()
        return PageReadMetrics(read_seconds=time.perf_counter() - started, logical_bytes=size, physical_bytes=size)

    def pinned_rows(self, start: int, stop: int) -> torch.Tensor | None:
        out = self.sink.out
        if not (out.is_pinned() and out.is_contiguous()):
            return None
        return out[start:stop]

    def close(self) -> torch.Tensor:
        return self.sink.out


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
        return _MemoryPageWriter(self, layout)


class _CallbackPageWriter(PageWriter):
    def __init__(self, callback: Callable[[PageDescriptor, torch.Tensor], object]) -> None:
        self.callback = callback
        self.pages_written = 0

    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        started = time.perf_counter()
        self.callback(page, data[: page.valid_tokens])
        self.pages_written += 1
        size = page.valid_tokens * data.shape[1] * data.shape[2] * data.element_size()
        return PageReadMetrics(read_seconds=time.perf_counter() - started, logical_bytes=size, physical_bytes=size)

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
