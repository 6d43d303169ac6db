"""DRAM K/V page cache (reference src/seqattn_core/paged/cache.py:24-229).

Same admission policy as the reference: a deterministic hot set (the first
``hot_fraction`` of the slots, owned by the first pages of the table, kept
once loaded) plus a rolling LRU region for every other page; the capacity is
``min(pages, capacity_bytes // slot_bytes)`` slots, registered as ``cache``
host memory.

Different storage: each slot holds a page's K/V record image (K rows at 0, V
rows at the record's ``v_offset``, INT8 scales after them) in page-locked
memory, so a hit is served by the copy engine straight from the slot and a
miss from an aligned store is read into its slot as one whole record (the
reference copies between an mmap region and a staging tensor on every hit and
insert).  Slots referenced by copies still in flight are never evicted.  For
INT8 pages a slot also holds the group scales expanded to one scale per
(row, head) for K and for V (``token_scale_layout``), the form the GPU
gather copies next to the rows.
"""

from __future__ import annotations

import math
import time
from collections import OrderedDict, deque
from collections.abc import Sequence
from dataclasses import dataclass

import torch

from ..storage.records import kv_record_pages
from .layout import KVLayout, PageDescriptor
from .memory_budget import HostMemoryPlan
from .slab import PinnedSlab


def token_scale_layout(record: PageDescriptor, layout: KVLayout) -> tuple[int, int, int]:
    """Slot offsets of the per-row K and V scales of an INT8 record, and the
    slot bytes it needs; (0, 0, record bytes) for other storage dtypes."""
    if layout.storage_dtype != "int8":
        return 0, 0, record.storage_bytes
    per_tensor = record.padded_tokens * layout.heads * 2
    k_offset = -(-record.storage_bytes // 256) * 256
    return k_offset, k_offset + per_tensor, k_offset + 2 * per_tensor


def expand_token_scales(raw: torch.Tensor, record: PageDescriptor, layout: KVLayout) -> None:
    """Fill the per-row scale areas of an INT8 slot image ``raw`` (uint8)
    from its ``[groups, heads]`` group scales: row j gets group j // quant_group_tokens."""
    k_offset, v_offset, _ = token_scale_layout(record, layout)
    rows, heads, group = record.padded_tokens, layout.heads, layout.quant_group_tokens
    groups = record.scale_bytes // (2 * heads)
    for scale_offset, token_offset in ((record.k_scale_offset, k_offset), (record.v_scale_offset, v_offset)):
        grouped = raw[scale_offset : scale_offset + record.scale_bytes].view(torch.float16).view(groups, heads)
        per_row = raw[token_offset : token_offset + rows * heads * 2].view(torch.float16).view(rows, heads)
        per_row.copy_(grouped.repeat_interleave(group, dim=0)[:rows])


@dataclass(frozen=True)
class CacheLookup:
    hit: bool
    seconds: float


class KVPageCache:
    """Two-region page cache over one page-locked slab of record slots."""

    def __init__(
        self,
        pages: Sequence[PageDescriptor],
        layout: KVLayout,
        *,
        capacity_bytes: int,
        hot_fraction: float,
        memory_plan: HostMemoryPlan,
        pinned: bool = True,
    ) -> None:
        self.layout = layout
        self.records = {r.page_id: r for r in kv_record_pages(pages, layout)}
        slot_bytes = max((token_scale_layout(r, layout)[2] for r in self.records.values()), default=0)
        count = min(len(pages), capacity_bytes // slot_bytes) if slot_bytes else 0
        self.memory_plan = memory_plan
        self.registered_bytes = 0
        self.slab = PinnedSlab(slot_bytes, 0, pinned=False)
        if count:
            probe = PinnedSlab(slot_bytes, 0, pinned=False)
            self.registered_bytes = count * probe.slot_bytes
            memory_plan.register("cache", self.registered_bytes)
            try:
                self.slab = PinnedSlab(slot_bytes, count, pinned=pinned)
            except BaseException:
                memory_plan.release("cache", self.registered_bytes)
                self.registered_bytes = 0
                raise
        self.slot_count = count
        hot = int(count * hot_fraction)
        if hot_fraction > 0 and count:
            hot = max(1, hot)
        self.hot_slot_count = min(count, hot)
        self._hot_slot = {p.page_id: i for i, p in enumerate(pages[: self.hot_slot_count])}
        self._hot_present: set[int] = set()
        self._rolling: OrderedDict[int, int] = OrderedDict()
        self._free = deque(range(self.hot_slot_count, count))
        self.hits = 0
        self.misses = 0
        self.peak_bytes = 0
        self._present = 0

    @property
    def hot_page_ids(self) -> frozenset[int]:
        return frozenset(self._hot_slot)

    @property
    def rolling_slot_count(self) -> int:
        return self.slot_count - self.hot_slot_count

    def _views(self, slot: int, page: PageDescriptor):
        record = self.records[page.page_id]
        raw = self.slab.bytes(slot)
        dtype = self.layout.storage_torch_dtype
        shape = (record.padded_tokens, self.layout.heads, self.layout.head_dim)
        k = raw[: record.k_bytes].view(dtype).view(shape)
        v = raw[record.v_offset : record.v_offset + record.v_bytes].view(dtype).view(shape)
        ks = vs = None
        if record.scale_bytes:
            groups = record.scale_bytes // (2 * self.layout.heads)
            ks = raw[record.k_scale_offset : record.k_scale_offset + record.scale_bytes].view(torch.float16)
            vs = raw[record.v_scale_offset : record.v_scale_offset + record.scale_bytes].view(torch.float16)
            ks, vs = ks.view(groups, self.layout.heads), vs.view(groups, self.layout.heads)
        return k, v, ks, vs

    def get(
        self,
        page: PageDescriptor,
        k_out: torch.Tensor,
        v_out: torch.Tensor,
        k_scales_out: torch.Tensor | None = None,
        v_scales_out: torch.Tensor | None = None,
    ) -> CacheLookup:
        """Copy a cached page into the given tensors (reference cache.py:87-127)."""
        slot, lookup = self.lookup(page)
        if slot is None:
            return lookup
        n = page.valid_tokens
        k, v, ks, vs = self._views(slot, page)
        k_out[:n].copy_(k[:n])
        v_out[:n].copy_(v[:n])
        if ks is not None:
            if k_scales_out is None or v_scales_out is None:
                raise ValueError("INT8 cache reads require scale buffers")
            groups = math.ceil(n / self.layout.quant_group_tokens)
            k_scales_out[:groups].copy_(ks[:groups])
            v_scales_out[:groups].copy_(vs[:groups])
        if k_out.shape[0] > n:
            k_out[n:].zero_()
            v_out[n:].zero_()
        return lookup

    def put(
        self,
        page: PageDescriptor,
        k: torch.Tensor,
        v: torch.Tensor,
        k_scales: torch.Tensor | None = None,
        v_scales: torch.Tensor | None = None,
    ) -> bool:
        """Insert a page by copy (reference cache.py:129-184); False when not admitted."""
        if self._present_slot(page) is not None:
            return True
        slot = self.reserve(page)
        if slot is None:
            return False
        n = page.valid_tokens
        kd, vd, ksd, vsd = self._views(slot, page)
        kd[:n].copy_(k[:n])
        vd[:n].copy_(v[:n])
        if ksd is not None:
            if k_scales is None or v_scales is None:
                raise ValueError("INT8 cache inserts require scale buffers")
            groups = math.ceil(n / self.layout.quant_group_tokens)
            ksd[:groups].copy_(k_scales[:groups])
            vsd[:groups].copy_(v_scales[:groups])
            expand_token_scales(self.slab.bytes(slot), self.records[page.page_id], self.layout)
        self.commit(page, slot)
        return True

    def _present_slot(self, page: PageDescriptor) -> int | None:
        if page.page_id in self._hot_slot:
            return self._hot_slot[page.page_id] if page.page_id in self._hot_present else None
        return self._rolling.get(page.page_id)

    def record(self, page: PageDescriptor) -> PageDescriptor:
        """The page with its record offsets (v_offset, scale offsets)."""
        return self.records[page.page_id]

    def lookup(self, page: PageDescriptor) -> tuple[int | None, CacheLookup]:
        """Slot holding ``page`` (hit) or None (miss)."""
        started = time.perf_counter()
        slot = None
        if page.page_id in self._hot_slot:
            if page.page_id in self._hot_present:
                slot = self._hot_slot[page.page_id]
        else:
            slot = self._rolling.get(page.page_id)
            if slot is not None:
                self._rolling.move_to_end(page.page_id)
        if slot is None:
            self.misses += 1
        else:
            self.hits += 1
        return slot, CacheLookup(slot is not None, time.perf_counter() - started)

    def reserve(self, page: PageDescriptor) -> int | None:
        """A slot to read a missed page into, or None when the page is not
        admitted (no cache, or every rolling slot is referenced)."""
        if not self.slot_count:
            return None
        if page.page_id in self._hot_slot:
            slot = self._hot_slot[page.page_id]
            if self.slab.held(slot):
                return None
            self.slab.wait_reusable(slot)
            return slot
        if self.hot_slot_count == self.slot_count:
            return None
        if self._free:
            slot = self._free.popleft()
            self.slab.wait_reusable(slot)
            return slot
        for victim, slot in self._rolling.items():
            if not self.slab.held(slot):
                del self._rolling[victim]
                self._present -= 1
                self.slab.wait_reusable(slot)
                return slot
        return None

    def commit(self, page: PageDescriptor, slot: int) -> None:
        """``slot`` now holds ``page``."""
        if page.page_id in self._hot_slot:
            if page.page_id not in self._hot_present:
                self._hot_present.add(page.page_id)
                self._present += 1
        else:
            self._rolling[page.page_id] = slot
            self._present += 1
        self.peak_bytes = max(self.peak_bytes, min(self._present, self.slot_count) * self.slab.slot_bytes)

    def abandon(self, page: PageDescriptor, slot: int) -> None:
        """A reserved slot was not filled (read failed)."""
        if page.page_id not in self._hot_slot:
            self._free.append(slot)

    def close(self) -> None:
        if self.registered_bytes:
            self.slab.close()
            self.memory_plan.release("cache", self.registered_bytes)
            self.registered_bytes = 0
        self.slot_count = 0

    def __enter__(self) -> KVPageCache:
        return self

    def __exit__(self, *_: object) -> None:
        self.close()


__all__ = ["CacheLookup", "KVPageCache", "expand_token_scales", "token_scale_layout"]
