"""FlashAttention-style entry points.

Names, signatures, validation messages and results follow the reference
(src/seqattn_core/api.py:15-113): packed ``[tokens, heads, head_dim]``
varlen inputs with ``cu_seqlens``, or dense ``[batch, seqlen, heads,
head_dim]`` inputs, in host DRAM, with the output returned in host DRAM.

What differs is the runner's lifetime.  A runner owns an HBM workspace and a
native pipeline (streams, events), which costs more to build than a small
attention call takes to run, so these functions keep the runner of the last
(plan, config) pair and reuse it while calls repeat it.  A lock serializes
calls on the shared runner, so concurrent callers stay correct.

Memory kept between calls: the cached runner's workspace, about the plan's
``estimated_workspace_bytes`` of HBM (at most the config's
``workspace_budget_bytes``), and its pipeline's streams and events.  The
transposed-V scratch of an HBM-resident call (as large as V) is dropped when
the call returns, and a call that raises drops the runner itself.
``clear_runner_cache()`` releases the runner; a different plan replaces it.
"""

from __future__ import annotations

import threading

import torch

from .config import StreamingAttentionConfig
from .planner import AttentionPlan, build_plan
from .stats import StreamingAttentionStats
from .streaming import StreamingAttentionRunner

_cache_lock = threading.Lock()
_cached: tuple[tuple, StreamingAttentionRunner] | None = None


def clear_runner_cache() -> None:
    """Release the runner kept by the last API call (its workspace and pipeline)."""
    global _cached
    with _cache_lock:
        if _cached is not None:
            _cached[1].close()
            _cached = None


def _run_cached(plan: AttentionPlan, config: StreamingAttentionConfig, call):
    global _cached
    key = (plan, config)
    with _cache_lock:
        if _cached is None or _cached[0] != key:
            if _cached is not None:
                _cached[1].close()
                _cached = None
            _cached = (key, StreamingAttentionRunner(plan, config))
        runner = _cached[1]
        try:
            result = call(runner)
        except BaseException:
            # A call that raised may have left work of its own on the
            # runner's buffers: drop the runner instead of reusing it.
            _cached = None
            runner.close()
            raise
        runner.release_resident_scratch()
        return result


def _longest_segment(cu_seqlens: torch.Tensor) -> int:
    bounds = cu_seqlens.to(dtype=torch.int64)
    if bounds.numel() < 2:
        return 0
    return int((bounds[1:] - bounds[:-1]).max().item())


def streaming_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int | None = None,
    max_seqlen_k: int | None = None,
    dropout_p: float = 0.0,
    softmax_scale: float | None = None,
    causal: bool = False,
    *,
    config: StreamingAttentionConfig | None = None,
    out: torch.Tensor | None = None,
    stats: StreamingAttentionStats | None = None,
    device: torch.device | str = "cuda",
    return_lse: bool = False,
):
    """Varlen attention over packed ``[total_tokens, heads, head_dim]`` host tensors.

    Q/K/V stay in host DRAM; the output is returned in host DRAM (or written
    into a device ``out``).  ``return_lse=True`` additionally returns the
    natural-log LSE ``[heads, total_q_tokens]``.
    """
    if dropout_p != 0:
        raise ValueError("seqattn V1 is inference-only and requires dropout_p=0")
    for cu, limit, which in ((cu_seqlens_q, max_seqlen_q, "q"), (cu_seqlens_k, max_seqlen_k, "k")):
        if limit is not None and _longest_segment(cu) > limit:
            raise ValueError(f"cu_seqlens_{which} exceeds max_seqlen_{which}")
    config = config if config is not None else StreamingAttentionConfig()
    plan = build_plan(
        q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=q.shape[2], dtype=q.dtype, device=device,
        max_q_tokens=q.shape[0], max_kv_tokens=k.shape[0], config=config,
    )
    return _run_cached(plan, config, lambda runner: runner(
        q, k, v, cu_seqlens_q, cu_seqlens_k,
        softmax_scale=softmax_scale, causal=causal, out=out, stats=stats, return_lse=return_lse,
    ))


def streaming_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dropout_p: float = 0.0,
    softmax_scale: float | None = None,
    causal: bool = False,
    *,
    config: StreamingAttentionConfig | None = None,
    out: torch.Tensor | None = None,
    stats: StreamingAttentionStats | None = None,
    device: torch.device | str = "cuda",
) -> torch.Tensor:
    """Dense batched wrapper over host ``[batch, seqlen, heads, head_dim]`` tensors:
    every batch entry is one segment of the packed varlen call."""
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("dense q, k, and v must use [batch, seqlen, heads, head_dim]")
    if q.shape[0] != k.shape[0] or k.shape != v.shape:
        raise ValueError("dense q/k/v batch and k/v shapes must match")
    batch, q_length, k_length = q.shape[0], q.shape[1], k.shape[1]
    packed = [t.flatten(0, 1) for t in (q, k, v)]
    segments = torch.arange(batch + 1, dtype=torch.int32)
    result = streaming_attn_varlen_func(
        *packed, segments * q_length, segments * k_length, q_length, k_length, dropout_p, softmax_scale, causal,
        config=config, out=None if out is None else out.flatten(0, 1), stats=stats, device=device,
    )
    return result.unflatten(0, (batch, q_length))


__all__ = [
    "AttentionPlan",
    "StreamingAttentionRunner",
    "clear_runner_cache",
    "streaming_attn_func",
    "streaming_attn_varlen_func",
]
