"""Compatibility module path of the projected pipeline (reference
src/seqattn/pipeline.py)."""

from .projection import (
    OutputProjector,
    ProjectedAttentionRunner,
    QKVProjector,
    streaming_projected_self_attention,
)

__all__ = [
    "OutputProjector",
    "ProjectedAttentionRunner",
    "QKVProjector",
    "streaming_projected_self_attention",
]
