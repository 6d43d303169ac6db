"""Import path of host-memory accounting kept from the reference (src/seqattn/host_memory.py)."""

from .paged.memory_budget import HostMemoryPlan, HostMemorySnapshot

__all__ = ["HostMemoryPlan", "HostMemorySnapshot"]
