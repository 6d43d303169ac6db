"""Device workspace and transfer pipeline handle.

Buffers follow CudaWorkspace (reference src/seqattn_core/streaming/workspace.py:8-50):
resident Q ``[q_chunk, Hq, D]``, a K/V ring of ``num_kv_buffers`` slots
``[kv_chunk, Hkv, D]``, FP32 state (running max/sum ``[q_chunk, Hq]``,
accumulator ``[q_chunk, Hq, D]``) and, in host output mode, raw output slots.
They are torch allocations, so the planner's budget accounts for all of them.
The ready/free events live in the native pipeline object bound to these
buffers; copies run on two torch streams handed to it and compute on torch's
current stream at creation.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _native
from ..planner import AttentionPlan


_COPY_STREAMS: dict[int, tuple[torch.cuda.Stream, torch.cuda.Stream]] = {}


def copy_streams(device: torch.device) -> tuple[torch.cuda.Stream, torch.cuda.Stream]:
    """The (H2D, D2H) copy streams of ``device``, created once per process.

    HIP maps streams onto a few hardware queues (GPU_MAX_HW_QUEUES, 4 by
    default) in creation order. A fresh pair per workspace walks that
    assignment, so after a few runners a copy stream can land on the compute
    stream's queue; its copies then wait behind kernels instead of
    overlapping them. Every workspace on a device shares this pair instead.
    Copies of different pipelines on the pair run in FIFO order; each
    pipeline's own events still order its copies against its kernels.
    """
    index = device.index if device.index is not None else torch.cuda.current_device()
    pair = _COPY_STREAMS.get(index)
    if pair is None:
        pair = (torch.cuda.Stream(device=index), torch.cuda.Stream(device=index))
        _COPY_STREAMS[index] = pair
    return pair


class CudaWorkspace:
    def __init__(self, plan: AttentionPlan) -> None:
        device = plan.device
        self.device = device
        self.q = torch.empty((plan.q_chunk_tokens, plan.q_heads, plan.head_dim), dtype=plan.dtype, device=device)
        self.k = [
            torch.empty((plan.kv_chunk_tokens, plan.kv_heads, plan.head_dim), dtype=plan.dtype, device=device)
            for _ in range(plan.num_kv_buffers)
        ]
        self.v = [torch.empty_like(t) for t in self.k]
        self.running_max = torch.empty((plan.q_chunk_tokens, plan.q_heads), dtype=torch.float32, device=device)
        self.running_sum = torch.empty_like(self.running_max)
        self.accumulator = torch.empty(
            (plan.q_chunk_tokens, plan.q_heads, plan.head_dim), dtype=torch.float32, device=device
        )
        self.output = (
            [torch.empty_like(self.q) for _ in range(plan.num_output_buffers)]
            if plan.output_mode == "host"
            else []
        )
        self.compute_stream = torch.cuda.current_stream(device)
        # Copy streams are torch streams (default priority) so torch's caching
        # allocator can track their uses of workspace and consumer buffers
        # (record_stream) for as long as those buffers live.
        self.h2d_stream, self.d2h_stream = copy_streams(device)

        lib = _native.lib()
        k_ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in self.k])
        v_ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in self.v])
        out_ptrs = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in self.output]) if self.output else None
        handle = ctypes.c_void_p()
        status = lib.sa_pipeline_create(
            ctypes.byref(handle),
            device.index if device.index is not None else torch.cuda.current_device(),
            self.q.data_ptr(), k_ptrs, v_ptrs, plan.num_kv_buffers,
            self.running_max.data_ptr(), self.running_sum.data_ptr(), self.accumulator.data_ptr(),
            out_ptrs, plan.num_output_buffers,
            plan.q_chunk_tokens, plan.kv_chunk_tokens, plan.q_heads, plan.kv_heads, plan.head_dim,
            _native.dtype_code(plan.dtype),
            self.h2d_stream.cuda_stream, self.d2h_stream.cuda_stream,
        )
        _native.check(status, "sa_pipeline_create")
        self._lib = lib
        self.handle = handle
        self.plan = plan
        self.resident_scratch: torch.Tensor | None = None

    def attach_resident_scratch(self, kv_tokens: int) -> None:
        """HBM-resident runs with head_dim 128: device scratch for V
        transposed per K/V head, [kv_heads, 128, kv_tokens padded to a
        multiple of 64] 16-bit elements, which the update kernel reads with
        half the LDS instructions.  Grown on demand and kept for later runs;
        outside the planner's workspace budget, like the resident inputs."""
        plan = self.plan
        if plan.head_dim != 128 or kv_tokens <= 0:
            return
        needed = plan.kv_heads * 128 * ((kv_tokens + 63) // 64 * 64) * 2
        if self.resident_scratch is None or self.resident_scratch.numel() < needed:
            # Allocated on the compute stream, where every run that reads it is
            # enqueued, so the caching allocator reuses a dropped buffer only
            # after those runs.
            self.resident_scratch = None
            with torch.cuda.stream(self.compute_stream):
                self.resident_scratch = torch.empty(needed, dtype=torch.uint8, device=self.device)
            status = self._lib.sa_pipeline_attach_resident_scratch(
                self.handle, self.resident_scratch.data_ptr(), self.resident_scratch.numel()
            )
            _native.check(status, "sa_pipeline_attach_resident_scratch")

    def close(self) -> None:
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            self._lib.sa_pipeline_destroy(handle)
            self.handle = None
        self.resident_scratch = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


__all__ = ["CudaWorkspace", "copy_streams"]
