"""Kernel boundary (reference src/seqattn_core/kernels/__init__.py).

The reference's Triton launch wrappers are replaced by calls into the gfx950
library through its C ABI; ``triton_is_available`` is kept as an alias of
``hip_is_available`` so capability checks in caller code keep working.
"""

from .streaming import (
    finalize_attention,
    hip_is_available,
    triton_is_available,
    update_attention_state,
    update_attention_state_int8,
)

__all__ = [
    "finalize_attention",
    "hip_is_available",
    "triton_is_available",
    "update_attention_state",
    "update_attention_state_int8",
]
