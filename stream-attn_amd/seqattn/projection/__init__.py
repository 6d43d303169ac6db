"""Projected self-attention: CPU hidden states -> QKV -> streamed attention ->
output projection (reference src/seqattn_core/projection/__init__.py)."""

from .api import streaming_projected_self_attention
from .runner import ProjectedAttentionRunner
from .types import OutputProjector, QKVProjector

__all__ = [
    "OutputProjector",
    "ProjectedAttentionRunner",
    "QKVProjector",
    "streaming_projected_self_attention",
]
