"""Torch-tensor wrappers of the chunk-update and finalize kernels.

``update_attention_state`` and ``finalize_attention`` keep the signatures of
the reference wrappers (src/seqattn_core/kernels/streaming.py:205-271 and
:345-371) and launch asynchronously on torch's current stream.  The launch
parameters block_m/block_n/num_warps/num_stages are accepted for
compatibility; the gfx950 kernel uses its own fixed tile (64 keys, and 384
queries per workgroup for head_dim 72-128, 256 for head_dim <= 64).  ``update_attention_state_int8``
(reference :274-342) dequantizes INT8 K/V inside the kernel.
``finalize_attention`` gains optional ``running_max`` / ``lse`` arguments
that write the natural-log LSE ``[heads, tokens]``.
"""

from __future__ import annotations

import torch

from .. import _native


def hip_is_available() -> bool:
    return _native.hip_is_available()


def triton_is_available() -> bool:
    """Alias of :func:`hip_is_available` (no Triton code exists in this package)."""
    return _native.hip_is_available()


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("kernel operands must be device tensors")
        if t.stride(-1) != 1:
            raise ValueError("kernel operands must have a unit stride in the last dimension")


def update_attention_state(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    running_max: torch.Tensor,
    running_sum: torch.Tensor,
    accumulator: torch.Tensor,
    *,
    q_tokens: int,
    kv_tokens: int,
    q_local_offset: int,
    kv_local_offset: int,
    causal_shift: int,
    softmax_scale: float,
    causal: bool,
    initialize: bool,
    block_m: int | None = None,
    block_n: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
) -> None:
    """Apply one K/V chunk to the FP32 online-softmax state of a Q block."""
    del block_m, block_n, num_warps, num_stages
    _require_device(q, k, v, accumulator)
    if running_max.stride() != running_sum.stride():
        raise ValueError("running_max and running_sum must share strides")
    if q_tokens > q.shape[0] or kv_tokens > k.shape[0] or kv_tokens > v.shape[0]:
        raise ValueError("q_tokens/kv_tokens exceed the operand buffers")
    if k.shape[1:] != v.shape[1:] or q.shape[2] != k.shape[2]:
        raise ValueError("q, k and v head_dim / kv_heads must agree")
    if accumulator.dtype != torch.float32 or running_max.dtype != torch.float32:
        raise ValueError("the attention state must be float32")
    flags = (_native.SA_FLAG_CAUSAL if causal else 0) | (
        _native.SA_FLAG_INITIALIZE if initialize else 0
    )
    stream = torch.cuda.current_stream(q.device).cuda_stream
    status = _native.lib().sa_update_attention_state(
        q.data_ptr(), k.data_ptr(), v.data_ptr(),
        running_max.data_ptr(), running_sum.data_ptr(), accumulator.data_ptr(),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        running_max.stride(0), running_max.stride(1),
        accumulator.stride(0), accumulator.stride(1),
        q_tokens, kv_tokens, q.shape[1], k.shape[1], q.shape[2],
        q_local_offset, kv_local_offset, causal_shift,
        float(softmax_scale), flags, _native.dtype_code(q.dtype), stream,
    )
    _native.check(status, "sa_update_attention_state")


def update_attention_state_int8(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_scales: torch.Tensor,
    v_scales: torch.Tensor,
    running_max: torch.Tensor,
    running_sum: torch.Tensor,
    accumulator: torch.Tensor,
    *,
    q_tokens: int,
    kv_tokens: int,
    q_local_offset: int,
    kv_local_offset: int,
    storage_token_offset: int,
    causal_shift: int,
    softmax_scale: float,
    causal: bool,
    initialize: bool,
    block_m: int | None = None,
    block_n: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
    quant_group_tokens: int = 64,
) -> None:
    """The chunk update with INT8 K/V (reference kernels/streaming.py:274-342).

    Key ``j`` of K/V head ``h`` is dequantized as
    ``q.dtype(float(k[j, h]) * float(k_scales[(storage_token_offset + j) //
    quant_group_tokens, h]))`` inside the kernel (same for V), so the result
    equals :func:`update_attention_state` on the dequantized K/V.
    """
    del block_m, block_n, num_warps, num_stages
    _require_device(q, k, v, accumulator)
    if k.dtype != torch.int8 or v.dtype != torch.int8:
        raise ValueError("quantized K/V buffers must use int8")
    if k_scales.dtype != torch.float16 or v_scales.dtype != torch.float16:
        raise ValueError("quantized K/V scales must use float16")
    if k_scales.device != q.device or v_scales.device != q.device:
        raise ValueError("quantized K/V scales must live on the query device")
    if k_scales.ndim != 2 or v_scales.ndim != 2:
        raise ValueError("quantized K/V scales must use [groups, kv_heads] layout")
    if running_max.stride() != running_sum.stride():
        raise ValueError("running_max and running_sum must share strides")
    if q_tokens > q.shape[0] or kv_tokens > k.shape[0] or kv_tokens > v.shape[0]:
        raise ValueError("q_tokens/kv_tokens exceed the operand buffers")
    if k.shape[1:] != v.shape[1:] or q.shape[2] != k.shape[2]:
        raise ValueError("q, k and v head_dim / kv_heads must agree")
    groups = (storage_token_offset + kv_tokens + quant_group_tokens - 1) // quant_group_tokens if kv_tokens else 0
    for scales in (k_scales, v_scales):
        if scales.shape[0] < groups or scales.shape[1] != k.shape[1]:
            raise ValueError("scale buffers do not cover the quantized K/V tokens")
    if accumulator.dtype != torch.float32 or running_max.dtype != torch.float32:
        raise ValueError("the attention state must be float32")
    flags = (_native.SA_FLAG_CAUSAL if causal else 0) | (
        _native.SA_FLAG_INITIALIZE if initialize else 0
    )
    stream = torch.cuda.current_stream(q.device).cuda_stream
    status = _native.lib().sa_update_attention_state_int8(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), k_scales.data_ptr(), v_scales.data_ptr(),
        running_max.data_ptr(), running_sum.data_ptr(), accumulator.data_ptr(),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        k_scales.stride(0), k_scales.stride(1), v_scales.stride(0), v_scales.stride(1),
        running_max.stride(0), running_max.stride(1),
        accumulator.stride(0), accumulator.stride(1),
        q_tokens, kv_tokens, q.shape[1], k.shape[1], q.shape[2],
        q_local_offset, kv_local_offset, storage_token_offset, causal_shift,
        float(softmax_scale), flags, _native.dtype_code(q.dtype), int(quant_group_tokens), stream,
    )
    _native.check(status, "sa_update_attention_state_int8")


def finalize_attention(
    accumulator: torch.Tensor,
    running_sum: torch.Tensor,
    output: torch.Tensor,
    *,
    q_tokens: int,
    running_max: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    lse_token_offset: int = 0,
) -> None:
    """``output = accumulator / running_sum`` (0 where the sum is 0).

    With ``lse`` (float32 ``[heads, >= lse_token_offset + q_tokens]``, unit
    token stride) and ``running_max``, also writes the natural-log LSE.
    """
    _require_device(accumulator, output)
    if lse is not None:
        if running_max is None:
            raise ValueError("lse output requires running_max")
        if lse.dtype != torch.float32 or lse.ndim != 2 or lse.stride(1) != 1:
            raise ValueError("lse must be a float32 [heads, tokens] tensor with unit token stride")
        if lse.shape[0] != output.shape[1] or lse.shape[1] < lse_token_offset + q_tokens:
            raise ValueError("lse is too small for the finalized rows")
    stream = torch.cuda.current_stream(output.device).cuda_stream
    status = _native.lib().sa_finalize_attention(
        accumulator.data_ptr(), None if running_max is None else running_max.data_ptr(),
        running_sum.data_ptr(), output.data_ptr(), None if lse is None else lse.data_ptr(),
        accumulator.stride(0), accumulator.stride(1),
        running_sum.stride(0), running_sum.stride(1),
        output.stride(0), output.stride(1),
        0 if lse is None else lse.stride(0), lse_token_offset,
        q_tokens, output.shape[1], output.shape[2], _native.dtype_code(output.dtype), stream,
    )
    _native.check(status, "sa_finalize_attention")


__all__ = [
    "finalize_attention",
    "hip_is_available",
    "triton_is_available",
    "update_attention_state",
    "update_attention_state_int8",
]
