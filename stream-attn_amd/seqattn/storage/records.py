"""Record layout of page stores (reference src/seqattn_core/storage/records.py:10-73).

A page record holds its padded rows: Q records ``[padded, H, D]``; K/V
records ``K [padded, Hkv, D] | V [padded, Hkv, D] | (INT8: K scales
[groups, Hkv] fp16 | V scales)``, each record padded to 4,096 bytes and
records laid back to back.  Identical to the reference so stores interchange.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

from ..paged.layout import KVLayout, PageDescriptor, TensorLayout, align_up, replace_page
from .direct_io import DIRECT_IO_ALIGNMENT


def q_record_pages(pages: Sequence[PageDescriptor], layout: TensorLayout) -> tuple[PageDescriptor, ...]:
    records, offset = [], 0
    for page in pages:
        payload = page.padded_tokens * layout.bytes_per_token
        storage = align_up(payload, DIRECT_IO_ALIGNMENT)
        records.append(replace_page(page, file_offset=offset, payload_bytes=payload,
                                    storage_bytes=storage, padding_bytes=storage - payload))
        offset += storage
    return tuple(records)


def kv_record_pages(pages: Sequence[PageDescriptor], layout: KVLayout) -> tuple[PageDescriptor, ...]:
    records, offset = [], 0
    for page in pages:
        tensor_bytes = page.padded_tokens * layout.storage_bytes_per_token
        payload = 2 * tensor_bytes
        k_scale_offset = v_scale_offset = scale_bytes = 0
        if layout.storage_dtype == "int8":
            scale_bytes = math.ceil(page.padded_tokens / layout.quant_group_tokens) * layout.heads * 2
            k_scale_offset = payload
            v_scale_offset = payload + scale_bytes
            payload += 2 * scale_bytes
        storage = align_up(payload, DIRECT_IO_ALIGNMENT)
        records.append(replace_page(
            page, file_offset=offset, payload_bytes=payload, storage_bytes=storage,
            padding_bytes=storage - payload, k_bytes=tensor_bytes, v_offset=tensor_bytes,
            v_bytes=tensor_bytes, k_scale_offset=k_scale_offset, v_scale_offset=v_scale_offset,
            scale_bytes=scale_bytes,
        ))
        offset += storage
    return tuple(records)


def expected_file_size(pages: Sequence[PageDescriptor]) -> int:
    return pages[-1].file_offset + pages[-1].storage_bytes if pages else 0


__all__ = ["expected_file_size", "kv_record_pages", "q_record_pages"]
