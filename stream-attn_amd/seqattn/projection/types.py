"""Callback types of the projected pipeline (reference
src/seqattn_core/projection/types.py:1-12).

``QKVProjector(hidden_tile, start, stop) -> (q, k, v)``: maps a device tile
``[tokens, hidden_features]`` of rows ``start:stop`` to device tensors
``[tokens, q_heads, head_dim]`` and ``[tokens, kv_heads, head_dim]`` (x2).

``OutputProjector(attention_tile, start, stop) -> projected``: maps a
finalized attention tile ``[tokens, q_heads * head_dim]`` in HBM to the
device rows written into ``out[start:stop]``.
"""

from collections.abc import Callable

import torch

QKVProjector = Callable[[torch.Tensor, int, int], tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
OutputProjector = Callable[[torch.Tensor, int, int], torch.Tensor]

__all__ = ["OutputProjector", "QKVProjector"]
