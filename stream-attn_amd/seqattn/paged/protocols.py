"""Page source / sink interfaces (reference src/seqattn_core/paged/protocols.py:13-82).

Same abstract methods and attributes as the reference, so sources and sinks
written against it plug in unchanged.  A reader fills caller-provided CPU
tensors; a writer receives one CPU page of output at a time.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Sequence

import torch

from .layout import KVLayout, PageDescriptor, PageReadMetrics, TensorLayout
from .memory_budget import HostMemoryPlan


class PageReader(ABC):
    @abstractmethod
    def read_q(self, page: PageDescriptor, out: torch.Tensor) -> PageReadMetrics:
        """Fill ``out[:page.valid_tokens]`` with the page's query rows (rows up
        to ``out.shape[0]`` beyond them are zeroed)."""

    @abstractmethod
    def read_kv(
        self,
        page: PageDescriptor,
        k_out: torch.Tensor,
        v_out: torch.Tensor,
        k_scales_out: torch.Tensor | None = None,
        v_scales_out: torch.Tensor | None = None,
    ) -> PageReadMetrics:
        """Fill the page's K and V rows in storage dtype (and INT8 scales)."""

    def close(self) -> None:
        return None

    def __enter__(self) -> PageReader:
        return self

    def __exit__(self, *_: object) -> None:
        self.close()


class PageSource(ABC):
    q_layout: TensorLayout | None
    kv_layout: KVLayout | None
    q_pages: tuple[PageDescriptor, ...]
    kv_pages: tuple[PageDescriptor, ...]
    cu_seqlens_q: tuple[int, ...] | None
    cu_seqlens_k: tuple[int, ...] | None
    direct_io: bool = False
    backing_kind: str = "memory"

    @abstractmethod
    def open_reader(self, memory_plan: HostMemoryPlan, queue_depth: int) -> PageReader:
        """A reader whose buffers are registered with ``memory_plan``."""


class PageWriter(ABC):
    @abstractmethod
    def write_page(self, page: PageDescriptor, data: torch.Tensor) -> PageReadMetrics:
        """Consume ``data[:page.valid_tokens]``; ``data`` is reused afterwards."""

    @abstractmethod
    def close(self) -> object:
        """Finish the output and return the run's result."""

    def abort(self) -> None:
        return None


class PageSink(ABC):
    backing_kind: str = "memory"

    @abstractmethod
    def open_writer(
        self,
        layout: TensorLayout,
        cu_seqlens: Sequence[int],
        pages: Sequence[PageDescriptor],
        memory_plan: HostMemoryPlan,
        queue_depth: int,
    ) -> PageWriter:
        """A writer for the query pages of ``layout``."""


__all__ = ["PageReader", "PageSink", "PageSource", "PageWriter"]
