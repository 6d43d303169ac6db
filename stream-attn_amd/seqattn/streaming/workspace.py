"""Device workspace and transfer pipeline handle.

Buffers follow CudaWorkspace (reference src/seqattn_core/streaming/workspace.py:8-50):
resident Q ``[q_chunk, Hq, D]``, a K/V ring of ``num_kv_buffers`` slots
``[kv_chunk, Hkv, D]``, FP32 state (running max/sum ``[q_chunk, Hq]``,
accumulator ``[q_chunk, Hq, D]``) and, in host output mode, raw output slots.
They are torch allocations, so the planner's budget accounts for all of them.
The ready/free events live in the native pipeline object bound to these
buffers; copies run on two torch streams handed to it and compute on torch's
current stream at creation.

A plan of the head-group schedule allocates its buffer sets instead: per set,
Q/output ``[max_q_tokens, Hq_group, D]``, K and V ``[max_kv_tokens,
Hkv_group, D]`` and, for head_dim 128, the transposed-V scratch of one
segment.  It has no Q block, ring or state buffers.
"""

from __future__ import annotations

import atexit
import ctypes
import weakref

import torch

from .. import _native
from ..planner import AttentionPlan


_COPY_STREAMS: dict[int, tuple[torch.cuda.Stream, torch.cuda.Stream]] = {}
# Page-locked staging of a head-group pipeline's output when the caller's out
# is pageable (row chunks of up to 64 MiB), outside the device budget.
HOST_STAGING_BYTES = 64 * 2**20
# Every workspace with a live native pipeline, so that all of them can be
# destroyed while the HIP runtime is still up (see close_all_workspaces).
_LIVE: "weakref.WeakSet[CudaWorkspace]" = weakref.WeakSet()


def close_all_workspaces() -> None:
    """Destroy every live pipeline and drop the shared copy streams.

    Registered with ``atexit``: it runs before the interpreter tears down
    modules and before the shared libraries' static destructors, so no
    pipeline (its events and side stream) and no scratch buffer is released
    after the HIP runtime has begun to shut down.
    """
    for workspace in list(_LIVE):
        try:
            workspace.close()
        except Exception:  # noqa: BLE001 - best effort at shutdown
            pass
    _COPY_STREAMS.clear()


atexit.register(close_all_workspaces)


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
        self.compute_stream = torch.cuda.current_stream(device)
        # Copy streams are torch streams (default priority) so torch's caching
        # allocator can track their uses of workspace and consumer buffers
        # (record_stream) for as long as those buffers live.
        self.h2d_stream, self.d2h_stream = copy_streams(device)
        self._lib = _native.lib()
        self.plan = plan
        self.resident_scratch: torch.Tensor | None = None
        self.host_staging: torch.Tensor | None = None
        self._staging_attached = False
        if plan.schedule == "head_groups":
            self._init_head_groups(plan)
        else:
            self._init_q_blocks(plan)
        _LIVE.add(self)

    def _init_head_groups(self, plan: AttentionPlan) -> None:
        device = self.device
        group = plan.q_heads // plan.kv_heads
        g = plan.head_group_kv_heads
        self.q, self.k, self.v, self.output = None, [], [], []
        self.running_max = self.running_sum = self.accumulator = None
        self.head_group_sets = [
            (
                torch.empty((plan.max_q_tokens, g * group, plan.head_dim), dtype=plan.dtype, device=device),
                torch.empty((plan.max_kv_tokens, g, plan.head_dim), dtype=plan.dtype, device=device),
                torch.empty((plan.max_kv_tokens, g, plan.head_dim), dtype=plan.dtype, device=device),
                torch.empty(plan.head_group_vt_bytes, dtype=torch.uint8, device=device)
                if plan.head_group_vt_bytes
                else None,
            )
            for _ in range(plan.head_group_sets)
        ]
        sets = self.head_group_sets

        def pointers(index):
            return (ctypes.c_void_p * 2)(*[s[index].data_ptr() for s in sets])

        vt = pointers(3) if plan.head_group_vt_bytes else None
        handle = ctypes.c_void_p()
        status = self._lib.sa_pipeline_create_head_groups(
            ctypes.byref(handle),
            device.index if device.index is not None else torch.cuda.current_device(),
            pointers(0), pointers(1), pointers(2), vt, plan.head_group_vt_bytes, len(sets),
            plan.max_q_tokens, plan.max_kv_tokens, g, plan.kv_chunk_tokens,
            plan.q_heads, plan.kv_heads, plan.head_dim, _native.dtype_code(plan.dtype),
            self.h2d_stream.cuda_stream, self.d2h_stream.cuda_stream,
        )
        _native.check(status, "sa_pipeline_create_head_groups")
        self.handle = handle

    def _init_q_blocks(self, plan: AttentionPlan) -> None:
        device = self.device
        self.head_group_sets = []
        self.q = torch.empty((plan.q_chunk_tokens, plan.q_heads, plan.head_dim), dtype=plan.dtype, device=device)
        self.k = [
            torch.empty((plan.kv_chunk_tokens, plan.kv_heads, plan.head_dim), dtype=plan.dtype, device=device)
            for _ in range(plan.num_kv_buffers)
        ]
        self.v = [torch.empty_like(t) for t in self.k]
        # FP32 state rows rounded up to the kernels' 16-row groups: the
        # pipeline stores the state group by group in the lanes' order.  The
        # at most 15 extra rows come out of the planner's fixed margin.
        state_rows = -(-plan.q_chunk_tokens // 16) * 16
        self.running_max = torch.empty((state_rows, plan.q_heads), dtype=torch.float32, device=device)
        self.running_sum = torch.empty_like(self.running_max)
        self.accumulator = torch.empty((state_rows, plan.q_heads, plan.head_dim), dtype=torch.float32, device=device)
        self.output = (
            [torch.empty_like(self.q) for _ in range(plan.num_output_buffers)]
            if plan.output_mode == "host"
            else []
        )
        lib = self._lib
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
        self.handle = handle

    def enable_trace_ranges(self) -> None:
        """Bracket each pipeline stage's enqueue with ROCm tracer ranges named
        like the reference's NVTX ranges (seqattn:q_h2d, kv_h2d, fused_update,
        fused_finalize, output_d2h)."""
        _native.check(self._lib.sa_pipeline_set_trace_ranges(self.handle, 1), "sa_pipeline_set_trace_ranges")

    def _attach(self, buffer: torch.Tensor | None) -> None:
        status = self._lib.sa_pipeline_attach_resident_scratch(
            self.handle, None if buffer is None else buffer.data_ptr(), 0 if buffer is None else buffer.numel()
        )
        _native.check(status, "sa_pipeline_attach_resident_scratch")

    def attach_resident_scratch(self, kv_tokens: int, limit_bytes: int | None = None) -> int:
        """HBM-resident runs with head_dim 128: device scratch for V
        transposed per K/V head, [kv_heads, 128, kv_tokens padded to a
        multiple of 64] 16-bit elements, which the update kernel reads with
        half the LDS instructions.  Grown on demand and kept for later runs;
        outside the planner's workspace budget, like the resident inputs.

        Returns the scratch bytes the next run will use, 0 when it reads V in
        place instead: ``limit_bytes`` caps the scratch (0 disables it), and
        an allocation that fails for lack of device memory also leaves the
        run on the in-place path, which gives the same results bit for bit.
        """
        plan = self.plan
        if plan.head_dim != 128 or kv_tokens <= 0:
            return 0
        needed = plan.kv_heads * 128 * ((kv_tokens + 63) // 64 * 64) * 2
        if self.resident_scratch is not None and self.resident_scratch.numel() >= needed:
            return needed
        if limit_bytes is not None and needed > limit_bytes:
            return 0
        # The pipeline must not hold the old buffer's address once it is dropped.
        if self.resident_scratch is not None:
            self._attach(None)
            self.resident_scratch = None
        try:
            # Allocated on the compute stream, where every run that reads it is
            # enqueued, so the caching allocator reuses a dropped buffer only
            # after those runs.
            with torch.cuda.stream(self.compute_stream):
                scratch = torch.empty(needed, dtype=torch.uint8, device=self.device)
        except torch.cuda.OutOfMemoryError:
            return 0
        self._attach(scratch)
        self.resident_scratch = scratch
        return needed

    def stage_output(self, enable: bool) -> None:
        """Head-group pipelines: copy the output through page-locked host
        staging (for a pageable out; strided copies into pageable memory are
        staged by the runtime row by row) or straight into the caller's
        page-locked rows."""
        if enable == self._staging_attached:
            return
        if enable and self.host_staging is None:
            self.host_staging = torch.empty(HOST_STAGING_BYTES, dtype=torch.uint8, pin_memory=True)
        buf = self.host_staging if enable else None
        status = self._lib.sa_pipeline_attach_host_staging(
            self.handle, None if buf is None else buf.data_ptr(), 0 if buf is None else buf.numel()
        )
        _native.check(status, "sa_pipeline_attach_host_staging")
        self._staging_attached = enable

    def release_resident_scratch(self) -> None:
        """Detach and drop the transposed-V scratch.  Runs already enqueued
        still read it: the buffer was allocated on the compute stream, so
        the caching allocator hands its memory out again only to work
        ordered after them."""
        if self.resident_scratch is not None:
            self._attach(None)
            self.resident_scratch = None

    def close(self) -> None:
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            # Work already enqueued on the compute stream records this
            # pipeline's events and reads its scratch: let it finish first.
            try:
                self.compute_stream.synchronize()
            except RuntimeError:
                pass
            self._lib.sa_pipeline_destroy(handle)
            self.handle = None
        self.resident_scratch = None
        self.host_staging = None
        _LIVE.discard(self)

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


__all__ = ["CudaWorkspace", "close_all_workspaces", "copy_streams"]
