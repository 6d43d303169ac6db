"""Page-locked host slabs carved into 4,096-byte aligned record slots.

One allocation per slab (``torch.empty(..., pin_memory=True)``, i.e.
hipHostMalloc), so the copy engines read every slot directly.  (O_DIRECT
cannot target this memory: the kernel refuses to map it for a direct
transfer, so direct-I/O reads go through an aligned bounce buffer.)  Each slot tracks the H2D copies
still reading it: ``hold`` counts fragments that reference the slot and are
not yet copied, ``release`` attaches the event that marks their copy done,
and ``wait_reusable`` blocks until no copy can still read the slot.
"""

from __future__ import annotations

import torch

SLOT_ALIGNMENT = 4096


def _align_up(value: int, alignment: int) -> int:
    return -(-value // alignment) * alignment


class PinnedSlab:
    def __init__(self, slot_bytes: int, count: int, *, pinned: bool) -> None:
        self.slot_bytes = _align_up(max(slot_bytes, 1), SLOT_ALIGNMENT)
        self.count = count
        self.nbytes = self.slot_bytes * count
        if count:
            self._raw = torch.empty(self.nbytes + SLOT_ALIGNMENT, dtype=torch.uint8, pin_memory=pinned)
            self._base = (-self._raw.data_ptr()) % SLOT_ALIGNMENT
        else:
            self._raw = torch.empty(0, dtype=torch.uint8)
            self._base = 0
        self._holds = [0] * count
        self._events: list[object | None] = [None] * count

    def bytes(self, slot: int) -> torch.Tensor:
        start = self._base + slot * self.slot_bytes
        return self._raw[start : start + self.slot_bytes]

    def address(self, slot: int) -> int:
        return self._raw.data_ptr() + self._base + slot * self.slot_bytes

    def hold(self, slot: int) -> None:
        self._holds[slot] += 1

    def release(self, slot: int, event) -> None:
        self._holds[slot] -= 1
        if self._holds[slot] < 0:
            raise RuntimeError("slot released more often than held")
        self._events[slot] = event

    def held(self, slot: int) -> bool:
        return self._holds[slot] > 0

    def wait_reusable(self, slot: int) -> None:
        if self._holds[slot]:
            raise RuntimeError("slot is still referenced by an un-issued copy")
        event = self._events[slot]
        if event is not None:
            event.synchronize()
            self._events[slot] = None

    def close(self) -> None:
        self._raw = torch.empty(0, dtype=torch.uint8)
        self.count = 0


__all__ = ["PinnedSlab", "SLOT_ALIGNMENT"]
