"""Symmetric INT8 K/V storage format (reference src/seqattn_core/quantization.py:8-49).

Per group of ``group_tokens`` consecutive tokens and per K/V head, values are
divided by ``amax / 127`` (1 where the group is all zero), rounded to nearest
even and clamped to [-127, 127]; the scale is stored as float16 in a
``[groups, heads]`` table.  The format must match the reference byte for byte
so INT8 stores written by either side read back the same.
"""

from __future__ import annotations

import math

import torch


def quantize_int8_per_token_group(
    source: torch.Tensor,
    quantized: torch.Tensor,
    scales: torch.Tensor,
    *,
    group_tokens: int = 64,
) -> None:
    """Quantize ``source [tokens, heads, head_dim]`` into ``quantized`` (int8)
    and ``scales [ceil(tokens / group_tokens), heads]`` (float16), in place."""
    if source.ndim != 3:
        raise ValueError("source must use [tokens, heads, head_dim] layout")
    if quantized.dtype != torch.int8 or quantized.shape != source.shape:
        raise ValueError("quantized must be an int8 tensor matching source")
    tokens, heads, _ = source.shape
    groups = math.ceil(tokens / group_tokens)
    if scales.dtype != torch.float16 or tuple(scales.shape) != (groups, heads):
        raise ValueError("scales must use float16 [groups, heads] layout")
    for g in range(groups):
        rows = slice(g * group_tokens, min((g + 1) * group_tokens, tokens))
        block = source[rows].float()
        step = block.abs().amax(dim=(0, 2)) / 127.0
        step = torch.where(step > 0, step, torch.ones_like(step))
        scales[g].copy_(step.to(torch.float16))
        quantized[rows].copy_(torch.round(block / step[None, :, None]).clamp_(-127, 127).to(torch.int8))


def dequantize_int8_per_token_group(
    quantized: torch.Tensor,
    scales: torch.Tensor,
    *,
    dtype: torch.dtype,
    group_tokens: int = 64,
) -> torch.Tensor:
    """Inverse of the storage format: ``q * scale`` in ``dtype``."""
    if quantized.ndim != 3 or quantized.dtype != torch.int8:
        raise ValueError("quantized must use int8 [tokens, heads, head_dim] layout")
    groups = math.ceil(quantized.shape[0] / group_tokens)
    if tuple(scales.shape) != (groups, quantized.shape[1]):
        raise ValueError("scale shape does not match quantized data")
    per_token = scales.float().repeat_interleave(group_tokens, dim=0)[: quantized.shape[0]]
    return (quantized.float() * per_token[:, :, None]).to(dtype)


__all__ = ["dequantize_int8_per_token_group", "quantize_int8_per_token_group"]
