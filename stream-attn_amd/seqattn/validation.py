"""Input checks (reference src/seqattn_core/validation.py:6-55; same messages)."""

from __future__ import annotations

import torch


def _segment_bounds(name: str, cu: torch.Tensor, total: int) -> list[int]:
    if cu.device.type != "cpu" or cu.ndim != 1 or cu.numel() < 2:
        raise ValueError(f"{name} must be a one-dimensional CPU tensor")
    bounds = cu.to(dtype=torch.int64).tolist()
    if bounds[0] != 0 or bounds[-1] != total:
        raise ValueError(f"{name} must span [0, {total}], got {bounds}")
    if any(b < a for a, b in zip(bounds[:-1], bounds[1:])):
        raise ValueError(f"{name} must be non-decreasing")
    return bounds


def validate_host_qkv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
) -> tuple[list[int], list[int]]:
    """Check packed [tokens, heads, head_dim] CPU inputs; return segment bounds."""
    if any(t.device.type != "cpu" for t in (q, k, v)):
        raise ValueError("seqattn expects CPU-backed q, k, and v tensors")
    return _validate_packed(q, k, v, cu_seqlens_q, cu_seqlens_k)


def validate_device_qkv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    device: torch.device,
) -> tuple[list[int], list[int]]:
    """Check HBM-resident packed inputs (all on ``device``); return segment bounds.

    Extension: the reference accepts CPU-backed inputs only (validation.py:13-14).
    """
    if any(t.device != device for t in (q, k, v)):
        raise ValueError(f"device-resident q, k, and v must all live on {device}")
    return _validate_packed(q, k, v, cu_seqlens_q, cu_seqlens_k)


def _validate_packed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
) -> tuple[list[int], list[int]]:
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k, and v must use packed [tokens, heads, head_dim] layout")
    if k.shape != v.shape:
        raise ValueError(f"k and v must have identical shapes, got {k.shape} and {v.shape}")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k/v must use the same head_dim")
    if q.shape[1] % k.shape[1]:
        raise ValueError("the number of query heads must be divisible by the number of KV heads")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, and v must use the same dtype")
    if not all(t.is_contiguous() for t in (q, k, v)):
        raise ValueError("q, k, and v must be contiguous")
    q_bounds = _segment_bounds("cu_seqlens_q", cu_seqlens_q, q.shape[0])
    k_bounds = _segment_bounds("cu_seqlens_k", cu_seqlens_k, k.shape[0])
    if len(q_bounds) != len(k_bounds):
        raise ValueError("cu_seqlens_q and cu_seqlens_k must describe the same batch size")
    for index in range(len(q_bounds) - 1):
        has_queries = q_bounds[index + 1] > q_bounds[index]
        has_keys = k_bounds[index + 1] > k_bounds[index]
        if has_queries and not has_keys:
            raise ValueError(f"sequence {index} has queries but no keys")
    return q_bounds, k_bounds


def require_pinned_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if not all(t.is_pinned() for t in (q, k, v)):
        raise ValueError(
            "asynchronous streaming requires pinned q, k, and v; call pin_memory() "
            "or set require_pinned=False for the synchronous fallback"
        )


__all__ = ["require_pinned_inputs", "validate_device_qkv", "validate_host_qkv"]
