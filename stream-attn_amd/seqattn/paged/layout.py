"""Page tables of paged sources (reference src/seqattn_core/paged/layout.py:9-206).

Descriptor fields, the dtype names and the page-splitting rule are the
reference's, so page tables and on-disk manifests written by either side
describe the same pages:

* a page never crosses a packed segment boundary;
* a page holds ``max(align, align_down(page_target_bytes // bytes_per_token,
  align))`` valid tokens except the last page of a segment, which holds the
  rest;
* ``padded_tokens`` rounds ``valid_tokens`` up to the token alignment
  (``block_n``), which is what a page's storage record is sized for.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import asdict, dataclass, replace

import torch

_DTYPES: dict[str, torch.dtype] = {
    "bf16": torch.bfloat16,
    "fp16": torch.float16,
    "fp32": torch.float32,
    "int8": torch.int8,
}
_NAMES = {dtype: name for name, dtype in _DTYPES.items()}


def align_up(value: int, alignment: int) -> int:
    if alignment <= 0:
        raise ValueError("alignment must be positive")
    return -(-value // alignment) * alignment


def align_down(value: int, alignment: int) -> int:
    if alignment <= 0:
        raise ValueError("alignment must be positive")
    return (value // alignment) * alignment


def dtype_name(dtype: torch.dtype) -> str:
    if dtype not in _NAMES:
        raise ValueError(f"unsupported dtype: {dtype}")
    return _NAMES[dtype]


def torch_dtype(name: str) -> torch.dtype:
    if name not in _DTYPES:
        raise ValueError(f"unsupported dtype name: {name}")
    return _DTYPES[name]


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


@dataclass(frozen=True)
class TensorLayout:
    """Packed ``[total_tokens, heads, head_dim]`` tensor of one dtype."""

    total_tokens: int
    heads: int
    head_dim: int
    dtype: str

    @property
    def torch_dtype(self) -> torch.dtype:
        return torch_dtype(self.dtype)

    @property
    def bytes_per_token(self) -> int:
        return self.heads * self.head_dim * _element_size(self.torch_dtype)

    def as_dict(self) -> dict[str, int | str]:
        return asdict(self)


@dataclass(frozen=True)
class KVLayout:
    """K/V pair layout: the caller's dtype and the dtype pages are stored in."""

    total_tokens: int
    heads: int
    head_dim: int
    source_dtype: str
    storage_dtype: str
    quant_group_tokens: int = 64

    @property
    def source_torch_dtype(self) -> torch.dtype:
        return torch_dtype(self.source_dtype)

    @property
    def storage_torch_dtype(self) -> torch.dtype:
        return torch_dtype(self.storage_dtype)

    @property
    def storage_bytes_per_token(self) -> int:
        return self.heads * self.head_dim * _element_size(self.storage_torch_dtype)

    def as_dict(self) -> dict[str, int | str]:
        return asdict(self)


@dataclass(frozen=True)
class PageDescriptor:
    """One page: a token range of one segment plus its storage record offsets."""

    page_id: int
    segment_id: int
    token_start: int
    segment_token_start: int
    valid_tokens: int
    padded_tokens: int
    file_offset: int = 0
    payload_bytes: int = 0
    storage_bytes: int = 0
    padding_bytes: int = 0
    k_bytes: int = 0
    v_offset: int = 0
    v_bytes: int = 0
    k_scale_offset: int = 0
    v_scale_offset: int = 0
    scale_bytes: int = 0

    @property
    def token_stop(self) -> int:
        return self.token_start + self.valid_tokens

    def as_dict(self) -> dict[str, int]:
        return asdict(self)

    @classmethod
    def from_dict(cls, payload: dict[str, int]) -> PageDescriptor:
        return cls(**payload)


@dataclass(frozen=True)
class PageReadMetrics:
    """Timing and byte counts of one page read or write."""

    read_seconds: float = 0.0
    quantization_seconds: float = 0.0
    logical_bytes: int = 0
    physical_bytes: int = 0
    simulated_io_seconds: float = 0.0
    simulated_service_seconds: float = 0.0
    simulated_queue_seconds: float = 0.0
    simulated_logical_bytes: int = 0
    simulated_physical_bytes: int = 0


def validate_cu_seqlens(cu_seqlens: torch.Tensor, total_tokens: int, name: str) -> list[int]:
    """Bounds of a CPU ``cu_seqlens`` tensor spanning ``[0, total_tokens]``."""
    if cu_seqlens.device.type != "cpu" or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"{name} must be a one-dimensional CPU tensor")
    bounds = [int(x) for x in cu_seqlens.tolist()]
    if bounds[0] != 0 or bounds[-1] != total_tokens:
        raise ValueError(f"{name} must span [0, {total_tokens}]")
    if any(b < a for a, b in zip(bounds, bounds[1:])):
        raise ValueError(f"{name} must be non-decreasing")
    return bounds


def build_page_descriptors(
    cu_seqlens: Sequence[int],
    *,
    bytes_per_token: int,
    page_target_bytes: int,
    token_alignment: int,
) -> tuple[PageDescriptor, ...]:
    """Split every segment into pages of about ``page_target_bytes``
    (reference paged/layout.py:147-175)."""
    if bytes_per_token <= 0 or page_target_bytes <= 0:
        raise ValueError("page sizing inputs must be positive")
    per_page = align_down(max(token_alignment, page_target_bytes // bytes_per_token), token_alignment)
    per_page = max(token_alignment, per_page)
    pages: list[PageDescriptor] = []
    bounds = [int(x) for x in cu_seqlens]
    for segment_id, (start, stop) in enumerate(zip(bounds, bounds[1:])):
        for local in range(0, stop - start, per_page):
            valid = min(per_page, stop - start - local)
            pages.append(
                PageDescriptor(
                    page_id=len(pages),
                    segment_id=segment_id,
                    token_start=start + local,
                    segment_token_start=local,
                    valid_tokens=valid,
                    padded_tokens=align_up(valid, token_alignment),
                )
            )
    return tuple(pages)


def pages_by_segment(
    pages: Sequence[PageDescriptor], segment_count: int
) -> tuple[tuple[PageDescriptor, ...], ...]:
    """Pages grouped by segment, keeping their order."""
    grouped: list[list[PageDescriptor]] = [[] for _ in range(segment_count)]
    for page in pages:
        if not 0 <= page.segment_id < segment_count:
            raise ValueError("page references an invalid segment")
        grouped[page.segment_id].append(page)
    return tuple(tuple(group) for group in grouped)


def replace_page(page: PageDescriptor, **changes: int) -> PageDescriptor:
    return replace(page, **changes)


__all__ = [
    "KVLayout",
    "PageDescriptor",
    "PageReadMetrics",
    "TensorLayout",
    "align_down",
    "align_up",
    "build_page_descriptors",
    "dtype_name",
    "pages_by_segment",
    "replace_page",
    "torch_dtype",
    "validate_cu_seqlens",
]
