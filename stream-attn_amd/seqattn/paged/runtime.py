"""Fixed-host-memory paged attention (reference src/seqattn_core/paged/runtime/runner.py:24-219,
paged/runtime/triton.py:28-310, paged/runtime/io.py:17-159, paged/runtime/contracts.py:16-60).

Same entry point, arguments, validation and stats as the reference's
``PagedAttentionRunner.run``.  The schedule is rebuilt for the MI355X path:

* query pages are packed into resident Q blocks of up to the planner's
  ``q_chunk_tokens`` (the reference keeps one page resident per K/V scan, so
  256-token pages mean one scan of all K/V per 256 queries);
* K/V pages are gathered into ring chunks of the planner's ``kv_chunk_tokens``
  by the native pipeline (``sa_pipeline_stream_kv_gather``), one H2D copy per
  page piece and one kernel launch per chunk, chunk boundaries aligned to
  multiples of the chunk within the segment as in tensor mode;
* page data reaches the copy engines from page-locked memory with no host
  copy where possible: the DRAM cache's slots are page-locked (hits are copied
  straight from the slot), misses from an aligned store are read as whole
  records into a cache slot or a staging slot, and page-locked caller tensors
  of a ``MemoryPageSource`` are read in place;
* K/V pages that the bottom-right causal mask hides from a whole Q block are
  neither read nor copied;
* ``run_with_device_output`` keeps the output in HBM (device-consumer mode,
  an extension: the reference requires host output for paged runs);
* INT8 pages cross PCIe as int8 rows plus one fp16 scale per (row, head) and
  are dequantized inside the update kernel, exactly as the reference's
  ``update_attention_state_int8`` does per page.

Host memory is accounted in a ``HostMemoryPlan`` with the reference's
categories; the page-locked cache slots are charged to ``cache``, staging
slots and the Q / output staging to ``pinned``.
"""

from __future__ import annotations

import ctypes
import math
import time
from collections import deque
from collections.abc import Callable
from concurrent.futures import Future, ThreadPoolExecutor
from contextlib import nullcontext
from dataclasses import replace

import torch

from .. import _native
from ..config import PagedAttentionConfig
from ..planner import build_plan
from ..stats import PagedAttentionStats
from ..storage.records import kv_record_pages
from ..streaming.backend import resolve_backend
from ..streaming.workspace import CudaWorkspace
from .cache import KVPageCache, expand_token_scales, token_scale_layout
from .layout import KVLayout, PageDescriptor, PageReadMetrics, TensorLayout, pages_by_segment, validate_cu_seqlens
from .memory_budget import HostMemoryPlan, HostMemorySnapshot
from .protocols import PageSink, PageSource
from .schedule import Fragment, FragmentQueue, QGroup, plan_q_groups
from .slab import PinnedSlab

_NATIVE_STORAGE = {"bf16", "fp16", "int8"}


def _backing_is_nvme(obj: object) -> bool:
    return getattr(obj, "backing_kind", "memory") == "nvme"


def validate_source_contract(
    q_source: PageSource,
    kv_source: PageSource,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    config: PagedAttentionConfig,
) -> tuple[TensorLayout, KVLayout, list[int], list[int]]:
    """Layouts and segment bounds of a source pair (reference paged/runtime/contracts.py:16-57)."""
    if q_source.q_layout is None:
        raise ValueError("q_source does not provide query pages")
    if kv_source.kv_layout is None:
        raise ValueError("kv_source does not provide K/V pages")
    q_layout, kv_layout = q_source.q_layout, kv_source.kv_layout
    q_bounds = validate_cu_seqlens(cu_seqlens_q, q_layout.total_tokens, "cu_seqlens_q")
    k_bounds = validate_cu_seqlens(cu_seqlens_k, kv_layout.total_tokens, "cu_seqlens_k")
    if len(q_bounds) != len(k_bounds):
        raise ValueError("query and K/V sources must describe the same batch size")
    if q_source.cu_seqlens_q is not None and tuple(q_bounds) != q_source.cu_seqlens_q:
        raise ValueError("cu_seqlens_q does not match q_source")
    if kv_source.cu_seqlens_k is not None and tuple(k_bounds) != kv_source.cu_seqlens_k:
        raise ValueError("cu_seqlens_k does not match kv_source")
    if q_layout.head_dim != kv_layout.head_dim or q_layout.heads % kv_layout.heads:
        raise ValueError("query and K/V head layouts are incompatible")
    if q_layout.dtype != kv_layout.source_dtype:
        raise ValueError("query and K/V source dtype must match")
    if kv_layout.storage_dtype != config.kv_storage_dtype:
        raise ValueError(
            "kv_source storage dtype does not match PagedAttentionConfig: "
            f"{kv_layout.storage_dtype} != {config.kv_storage_dtype}"
        )
    for index, (q0, q1, k0, k1) in enumerate(zip(q_bounds, q_bounds[1:], k_bounds, k_bounds[1:])):
        if q1 > q0 and k1 == k0:
            raise ValueError(f"sequence {index} has queries but no keys")
    for source in {id(q_source): q_source, id(kv_source): kv_source}.values():
        if _backing_is_nvme(source) and source.direct_io != config.direct_io:
            raise ValueError(
                "NVMe source direct_io mode must match PagedAttentionConfig; "
                "buffered fallback is never implicit"
            )
    return q_layout, kv_layout, q_bounds, k_bounds


class _StageRing:
    """Page-locked record slots for K/V pages that are not cached."""

    def __init__(self, slot_bytes: int, count: int, pinned: bool) -> None:
        self.slab = PinnedSlab(slot_bytes, count, pinned=pinned)
        self.free = deque(range(count))

    def release(self, slot: int, event) -> None:
        self.slab.release(slot, event)
        if not self.slab.held(slot):
            self.free.append(slot)


class _Load:
    """One K/V page on its way into page-locked memory."""

    __slots__ = ("page", "future", "k_address", "v_address", "owner", "commit_slot", "ks_address", "vs_address")

    def __init__(self, page, future, k_address, v_address, owner, commit_slot=None, ks_address=0, vs_address=0):
        self.page = page
        self.future = future
        self.k_address = k_address
        self.v_address = v_address
        self.owner = owner
        self.commit_slot = commit_slot
        self.ks_address = ks_address
        self.vs_address = vs_address


class PagedAttentionRunner:
    """Fixed-host-memory paged attention runtime for memory or NVMe sources."""

    def __init__(self, config: PagedAttentionConfig | None = None, *, device: torch.device | str = "cuda") -> None:
        self.config = PagedAttentionConfig() if config is None else config
        self.device = torch.device(device)
        self._nvtx = False

    def _range(self, name: str):
        return torch.cuda.nvtx.range(name) if self._nvtx else nullcontext()

    @torch.no_grad()
    def run(
        self,
        q_source: PageSource,
        kv_source: PageSource,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        output_sink: PageSink,
        *,
        config: PagedAttentionConfig | None = None,
        softmax_scale: float | None = None,
        causal: bool = False,
        stats: PagedAttentionStats | None = None,
        lse_out: torch.Tensor | None = None,
    ) -> object:
        """Attention of the query pages against the K/V pages, written page by
        page to ``output_sink``; returns the writer's ``close()`` result.
        ``lse_out`` (extension): float32 device tensor ``[q_heads, total_q]``."""
        config = self.config if config is None else config
        config.validate()
        if _backing_is_nvme(output_sink) and getattr(output_sink, "direct_io", None) != config.direct_io:
            raise ValueError("NVMe output sink direct_io mode must match PagedAttentionConfig")
        if config.attention.output_mode != "host":
            raise ValueError("paged output sinks require attention output_mode='host'")
        return self._execute(q_source, kv_source, cu_seqlens_q, cu_seqlens_k, config, softmax_scale, causal,
                             stats, sink=output_sink, lse=lse_out)

    @torch.no_grad()
    def run_with_device_output(
        self,
        q_source: PageSource,
        kv_source: PageSource,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        *,
        out: torch.Tensor | None = None,
        output_transform: Callable[[torch.Tensor, int, int], torch.Tensor] | None = None,
        config: PagedAttentionConfig | None = None,
        softmax_scale: float | None = None,
        causal: bool = False,
        stats: PagedAttentionStats | None = None,
        lse_out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Device-consumer mode: the output stays in HBM.

        Without ``output_transform`` each Q block is finalized straight into
        ``out[rows]`` (allocated ``[total_q, q_heads, head_dim]`` on the
        device when omitted).  With it, ``output_transform(tile [rows,
        q_heads * head_dim], start, stop)`` runs on the compute stream and its
        result is copied into ``out[start:stop]``.
        """
        config = self.config if config is None else config
        config.validate()
        return self._execute(q_source, kv_source, cu_seqlens_q, cu_seqlens_k, config, softmax_scale, causal,
                             stats, device_out=out, transform=output_transform, lse=lse_out,
                             device_mode=True)

    # ------------------------------------------------------------------ helpers

    @staticmethod
    def _record_memory_stats(stats: PagedAttentionStats, snapshot: HostMemorySnapshot) -> None:
        stats.operator_host_allocated_bytes = snapshot.operator_host_allocated_bytes
        stats.operator_host_peak_bytes = snapshot.operator_host_peak_bytes
        stats.pinned_peak_bytes = snapshot.pinned_peak_bytes
        stats.direct_io_bounce_peak_bytes = snapshot.direct_io_bounce_peak_bytes
        stats.dram_cache_peak_bytes = snapshot.dram_cache_peak_bytes
        stats.host_memory_budget_bytes = snapshot.host_memory_budget_bytes

    @staticmethod
    def _account_read(stats: PagedAttentionStats, metrics: PageReadMetrics, is_nvme: bool) -> None:
        stats.quantization_seconds += metrics.quantization_seconds
        if is_nvme:
            stats.nvme_read_seconds += metrics.read_seconds
            stats.nvme_logical_read_bytes += metrics.logical_bytes
            stats.nvme_physical_read_bytes += metrics.physical_bytes
        stats.simulated_read_seconds += metrics.simulated_io_seconds
        stats.simulated_read_service_seconds += metrics.simulated_service_seconds
        stats.simulated_read_queue_seconds += metrics.simulated_queue_seconds
        stats.simulated_logical_read_bytes += metrics.simulated_logical_bytes
        stats.simulated_physical_read_bytes += metrics.simulated_physical_bytes

    @staticmethod
    def _account_write(stats: PagedAttentionStats, metrics: PageReadMetrics, is_nvme: bool) -> None:
        stats.output_write_seconds += metrics.read_seconds
        if is_nvme:
            stats.nvme_write_seconds += metrics.read_seconds
            stats.nvme_logical_write_bytes += metrics.logical_bytes
            stats.nvme_physical_write_bytes += metrics.physical_bytes
        stats.simulated_write_seconds += metrics.simulated_io_seconds
        stats.simulated_write_service_seconds += metrics.simulated_service_seconds
        stats.simulated_write_queue_seconds += metrics.simulated_queue_seconds
        stats.simulated_logical_write_bytes += metrics.simulated_logical_bytes
        stats.simulated_physical_write_bytes += metrics.simulated_physical_bytes

    # ---------------------------------------------------------------- execution

    def _execute(self, q_source, kv_source, cu_seqlens_q, cu_seqlens_k, config, softmax_scale, causal, stats,
                 *, sink=None, device_out=None, transform=None, lse=None, device_mode=False):
        self._nvtx = bool(config.attention.enable_nvtx and torch.cuda.is_available())
        q_layout, kv_layout, q_bounds, k_bounds = validate_source_contract(
            q_source, kv_source, cu_seqlens_q, cu_seqlens_k, config)
        if kv_layout.storage_dtype not in _NATIVE_STORAGE:
            raise ValueError("the HIP paged backend supports bf16, fp16 and int8 K/V storage, not "
                             f"{kv_layout.storage_dtype}")
        if kv_layout.storage_dtype == "int8" and (q_layout.head_dim % 16 or q_layout.head_dim > 128):
            raise ValueError("INT8 K/V pages need head_dim a multiple of 16 and at most 128")
        attention = config.attention
        if attention.schedule == "head_groups":
            raise ValueError("paged runs gather pages into Q blocks: they need schedule='q_blocks'")
        attention = replace(attention, schedule="q_blocks")  # "auto" plans Q blocks here
        if device_mode:
            attention = replace(attention, output_mode="device_consumer")
        plan = build_plan(
            q_heads=q_layout.heads, kv_heads=kv_layout.heads, head_dim=q_layout.head_dim,
            dtype=q_layout.torch_dtype, device=self.device, max_q_tokens=q_layout.total_tokens,
            max_kv_tokens=kv_layout.total_tokens, config=attention,
        )
        backend = resolve_backend(attention.backend, plan.dtype, plan.device, head_dim=plan.head_dim)
        device = plan.device if plan.device.index is not None else torch.device("cuda", torch.cuda.current_device())
        total_q = q_layout.total_tokens
        if device_mode:
            if device_out is None:
                device_out = torch.empty((total_q, q_layout.heads, q_layout.head_dim), dtype=q_layout.torch_dtype,
                                         device=device)
            if device_out.device != device or device_out.shape[0] != total_q or not device_out.is_contiguous():
                raise ValueError("out must be a contiguous device tensor with one row per query token")
            if transform is None and (device_out.shape[1:] != (q_layout.heads, q_layout.head_dim)
                                      or device_out.dtype != q_layout.torch_dtype):
                raise ValueError("out must match the query layout")
        if lse is not None and (lse.device != device or lse.dtype != torch.float32 or lse.ndim != 2
                                or lse.shape[0] != q_layout.heads or lse.shape[1] < total_q or lse.stride(1) != 1):
            raise ValueError("lse_out must be a float32 device tensor [q_heads, >= total_q_tokens]")

        stats = PagedAttentionStats() if stats is None else stats
        stats.backend = backend
        stats.kv_storage_dtype = kv_layout.storage_dtype
        stats.q_chunk_tokens = plan.q_chunk_tokens
        stats.kv_chunk_tokens = plan.kv_chunk_tokens
        stats.estimated_workspace_bytes = plan.estimated_workspace_bytes
        scale = plan.head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
        segments = len(q_bounds) - 1
        q_pages_by_segment = pages_by_segment(q_source.q_pages, segments)
        kv_pages_by_segment = pages_by_segment(kv_source.kv_pages, segments)

        memory_plan = HostMemoryPlan(
            total_budget_bytes=config.host_memory_budget_bytes,
            pinned_limit_bytes=config.pinned_staging_budget_bytes,
            bounce_limit_bytes=config.direct_io_bounce_budget_bytes,
            metadata_margin_bytes=config.metadata_margin_bytes,
        )
        state = _RunState()
        started = time.perf_counter()
        completed = None
        try:
            state.open(self, q_source, kv_source, sink, memory_plan, config, q_layout, kv_layout, plan, q_bounds,
                       device_mode, device)
            with self._range("seqattn_paged:execute"), torch.cuda.device(device):
                self._schedule(state, plan, config, q_layout, kv_layout, q_bounds, k_bounds, q_pages_by_segment,
                               kv_pages_by_segment, scale, causal, stats, device_out, transform, lse)
            state.finish_writes(self, stats)
            result = device_out if device_mode else state.writer.close()
            state.writer = None
            cache = state.cache
            stats.cache_hits += cache.hits
            stats.cache_misses += cache.misses
            lookups = stats.cache_hits + stats.cache_misses
            stats.cache_hit_ratio = stats.cache_hits / lookups if lookups else 0.0
            completed = memory_plan.snapshot()
            stats.wall_seconds += time.perf_counter() - started
            self._record_memory_stats(stats, completed)
            return result
        except BaseException:
            state.abort()
            raise
        finally:
            state.close()
            self._record_memory_stats(stats, completed or memory_plan.snapshot())

    def _schedule(self, state, plan, config, q_layout, kv_layout, q_bounds, k_bounds, q_pages_by_segment,
                  kv_pages_by_segment, scale, causal, stats, device_out, transform, lse):
        lib = _native.lib()
        ws = state.workspace
        handle = ws.handle
        compute = ws.compute_stream
        compute_ptr = compute.cuda_stream
        native = _native.PipelineStats()
        native_ref = ctypes.byref(native)
        q_row_bytes = q_layout.bytes_per_token
        kv_row_bytes = kv_layout.storage_bytes_per_token
        lse_ptr = None if lse is None else lse.data_ptr()
        lse_stride = 0 if lse is None else lse.stride(0)
        depth = max(1, config.io_queue_depth)
        kernel_start = torch.cuda.Event(enable_timing=True)
        kernel_end = torch.cuda.Event(enable_timing=True)
        kernel_start.record(compute)
        # Every Q block in execution order, so the next block's query pages can
        # be read while the current block streams its K/V.
        blocks = []
        group_index = 0
        for segment, q_pages in enumerate(q_pages_by_segment):
            if q_bounds[segment + 1] == q_bounds[segment]:
                continue
            for group in plan_q_groups(q_pages, state.q_rows):
                for position, block in enumerate(group.blocks):
                    blocks.append((segment, group, group_index, block, position == len(group.blocks) - 1))
                group_index += 1

        for index, (segment, group, group_id, block, group_end) in enumerate(blocks):
            q0 = q_bounds[segment]
            k0, k1 = k_bounds[segment], k_bounds[segment + 1]
            shift = (k1 - k0) - (q_bounds[segment + 1] - q0)
            out_slot = group_id % max(1, len(state.out_stage))
            if state.out_stage and block.group_offset == 0:
                state.wait_out_slot(out_slot, self, stats)
            n = block.rows
            global_start = q0 + block.segment_start
            # Q block -> resident Q buffer.
            with self._range("seqattn_paged:q_h2d"):
                q_address = state.load_q_rows(self, block, q_row_bytes, stats, global_start)
                _native.check(lib.sa_pipeline_load_q(handle, q_address, n, compute_ptr, native_ref),
                              "sa_pipeline_load_q")
                state.q_loaded()
            stats.q_chunks += 1
            stats.kv_page_scans += 1
            following = blocks[index + 1][3] if index + 1 < len(blocks) else None
            prefetch = (lambda b=following: state.prefetch_q(b)) if following is not None else None
            # K/V pages -> gathered ring chunks -> update launches.
            with self._range("seqattn_paged:kv_scan"):
                self._scan(state, lib, handle, compute_ptr, native_ref, plan, kv_pages_by_segment[segment], k0,
                           n, block.segment_start, shift, scale, causal, depth, kv_row_bytes, stats, prefetch)
            # Finalize and deliver the block's output.
            with self._range("seqattn_paged:finalize"):
                self._deliver(state, lib, handle, compute, compute_ptr, native_ref, block, group, out_slot, n,
                              global_start, q_row_bytes, device_out, transform, lse_ptr, lse_stride, stats)
            if state.out_stage and group_end:
                state.write_group(self, group, out_slot, stats)
        kernel_end.record(compute)
        kernel_end.synchronize()
        stats.gpu_kernel_seconds += kernel_start.elapsed_time(kernel_end) / 1e3
        _native.check(lib.sa_pipeline_synchronize(handle), "sa_pipeline_synchronize")
        stats.h2d_bytes += native.h2d_bytes
        stats.d2h_bytes += native.d2h_bytes
        stats.state_spills += native.kv_tiles

    def _scan(self, state, lib, handle, compute_ptr, native_ref, plan, kv_pages, k0, q_tokens, q_local_offset,
              shift, scale, causal, depth, kv_row_bytes, stats, prefetch=None):
        """Stream one segment's K/V pages through the ring for one Q block."""
        if causal:
            visible_end = q_local_offset + q_tokens + shift
            pages = [p for p in kv_pages if p.segment_token_start < visible_end] or list(kv_pages[:1])
        else:
            pages = list(kv_pages)
        int8 = state.int8
        queue = FragmentQueue(kv_row_bytes, state.scale_row_bytes if int8 else 0)
        initialize = ctypes.c_int32(1)
        issued = 0
        kv_chunk = plan.kv_chunk_tokens

        def issue(rows: int) -> None:
            nonlocal issued
            pieces, finished = queue.take(rows)
            count = len(pieces)
            k_ptrs = (ctypes.c_void_p * count)(*[p[0] for p in pieces])
            v_ptrs = (ctypes.c_void_p * count)(*[p[1] for p in pieces])
            lengths = (ctypes.c_int32 * count)(*[p[2] for p in pieces])
            copy_started = time.perf_counter()
            if int8:
                ks_ptrs = (ctypes.c_void_p * count)(*[p[3] for p in pieces])
                vs_ptrs = (ctypes.c_void_p * count)(*[p[4] for p in pieces])
                _native.check(
                    lib.sa_pipeline_stream_kv_gather_int8(
                        handle, k_ptrs, v_ptrs, ks_ptrs, vs_ptrs, lengths, count, issued, ctypes.byref(initialize),
                        q_tokens, q_local_offset, shift, float(scale), int(bool(causal)), compute_ptr, native_ref),
                    "sa_pipeline_stream_kv_gather_int8")
            else:
                _native.check(
                    lib.sa_pipeline_stream_kv_gather(
                        handle, k_ptrs, v_ptrs, lengths, count, issued, ctypes.byref(initialize), q_tokens,
                        q_local_offset, shift, float(scale), int(bool(causal)), compute_ptr, native_ref),
                    "sa_pipeline_stream_kv_gather")
            stats.pinned_copy_seconds += time.perf_counter() - copy_started
            event = torch.cuda.Event()
            event.record(state.workspace.h2d_stream)
            for owner in finished:
                state.release(owner, event)
            issued += rows

        loads: deque[_Load] = deque()
        position = 0
        for _ in range(min(depth, len(pages))):
            loads.append(state.submit_kv(self, pages[position], k0, issue, queue, stats))
            position += 1
        if prefetch is not None:
            prefetch()
        while loads:
            load = loads.popleft()
            if load.future is not None:
                wait_started = time.perf_counter()
                metrics = load.future.result()
                stats.io_queue_wait_seconds += time.perf_counter() - wait_started
                self._account_read(stats, metrics, state.kv_is_nvme)
            if load.commit_slot is not None:
                state.cache.commit(load.page, load.commit_slot)
            queue.push(Fragment(load.k_address, load.v_address, load.page.valid_tokens, load.owner,
                                load.ks_address, load.vs_address))
            stats.kv_pages += 1
            if queue.rows >= kv_chunk:
                issue((queue.rows // kv_chunk) * kv_chunk)
            if position < len(pages):
                loads.append(state.submit_kv(self, pages[position], k0, issue, queue, stats))
                position += 1
        if queue.rows:
            issue(queue.rows)
        if initialize.value:
            _native.check(
                lib.sa_pipeline_stream_kv_span(handle, None, None, 0, 0, ctypes.byref(initialize), q_tokens,
                                               q_local_offset, shift, float(scale), int(bool(causal)),
                                               compute_ptr, native_ref),
                "sa_pipeline_stream_kv_span")

    def _deliver(self, state, lib, handle, compute, compute_ptr, native_ref, block, group, out_slot, n,
                 global_start, q_row_bytes, device_out, transform, lse_ptr, lse_stride, stats):
        ws = state.workspace
        if device_out is not None and transform is None:
            target = device_out[global_start : global_start + n]
            _native.check(lib.sa_pipeline_finalize_into(handle, target.data_ptr(), target.stride(0),
                                                        target.stride(1), n, lse_ptr, lse_stride, global_start,
                                                        compute_ptr), "sa_pipeline_finalize_into")
            return
        if device_out is not None:
            _native.check(lib.sa_pipeline_finalize(handle, -1, n, lse_ptr, lse_stride, global_start, compute_ptr),
                          "sa_pipeline_finalize")
            with torch.cuda.stream(compute):
                tile = transform(ws.q[:n].reshape(n, -1), global_start, global_start + n)
                destination = device_out[global_start : global_start + n]
                if tile.device != device_out.device or tile.shape != destination.shape or tile.dtype != destination.dtype:
                    raise ValueError("output_transform result must match the output slice on the device")
                destination.copy_(tile)
            _native.check(lib.sa_pipeline_release_q(handle, compute_ptr), "sa_pipeline_release_q")
            return
        # Host output: finalize into a device output slot, then D2H.
        slot = state.next_device_slot()
        _native.check(lib.sa_pipeline_finalize(handle, slot, n, lse_ptr, lse_stride, global_start, compute_ptr),
                      "sa_pipeline_finalize")
        source = ws.output[slot][:n]
        if state.direct_out is not None:
            destination = state.direct_out[global_start : global_start + n]
        else:
            destination = state.out_stage[out_slot][block.group_offset : block.group_offset + n]
        _native.check(lib.sa_pipeline_d2h(handle, destination.data_ptr(), source.data_ptr(), n * q_row_bytes,
                                          slot, 0, compute_ptr, native_ref), "sa_pipeline_d2h")
        source.record_stream(ws.d2h_stream)


class _RunState:
    """Buffers, readers and bookkeeping of one paged run."""

    def __init__(self) -> None:
        self.q_reader = self.kv_reader = self.writer = None
        self.cache = None
        self.stages = None
        self.pool = None
        self.workspace = None
        self.q_stage = None
        self.q_page_buffer = None
        self.out_stage: list[torch.Tensor] = []
        self.out_futures: list[list[Future]] = []
        self.out_events: list[object | None] = []
        self.direct_out = None
        self.zero_copy_kv = None
        self.zero_copy_q = None
        self.pinned_registered = 0
        self.memory_plan = None
        self.q_event = None
        self.q_event_pending = False
        self.q_reads = None
        self.device_slot = 0
        self.kv_is_nvme = False
        self.q_is_nvme = False
        self.out_is_nvme = False
        self.q_rows = 0
        self.int8 = False
        self.kv_layout = None
        self.scale_row_bytes = 0
        self.scale_ring: list[torch.Tensor] = []

    def open(self, runner, q_source, kv_source, sink, memory_plan, config, q_layout, kv_layout, plan, q_bounds,
             device_mode, device):
        self.memory_plan = memory_plan
        self.kv_layout = kv_layout
        self.int8 = kv_layout.storage_dtype == "int8"
        self.scale_row_bytes = kv_layout.heads * 2
        self.kv_is_nvme = _backing_is_nvme(kv_source)
        self.q_is_nvme = _backing_is_nvme(q_source)
        self.out_is_nvme = sink is not None and _backing_is_nvme(sink)
        depth = max(1, config.io_queue_depth)
        if q_source is kv_source:
            self.q_reader = self.kv_reader = q_source.open_reader(memory_plan, depth)
        else:
            self.q_reader = q_source.open_reader(memory_plan, 1)
            self.kv_reader = kv_source.open_reader(memory_plan, depth)
        if sink is not None:
            self.writer = sink.open_writer(q_layout, q_bounds, q_source.q_pages, memory_plan,
                                           config.num_output_buffers)
        pinned = torch.cuda.is_available()

        # Zero-copy paths over page-locked caller memory.
        if hasattr(kv_source, "pinned_kv_rows") and kv_source.pinned_kv_rows(0, 0) is not None:
            self.zero_copy_kv = kv_source
        if hasattr(q_source, "pinned_q_rows") and q_source.pinned_q_rows(0, 0) is not None:
            self.zero_copy_q = q_source
        if self.writer is not None and hasattr(self.writer, "pinned_rows"):
            self.direct_out = self.writer.pinned_rows(0, q_layout.total_tokens)

        # DRAM cache (not for memory-backed sources, as in the reference).
        capacity = min(memory_plan.cache_limit_bytes,
                       max(0, memory_plan.total_budget_bytes - memory_plan.current_bytes))
        if getattr(kv_source, "backing_kind", "memory") == "memory":
            capacity = 0
        self.cache = KVPageCache(kv_source.kv_pages, kv_layout, capacity_bytes=capacity,
                                 hot_fraction=config.cache_hot_fraction, memory_plan=memory_plan, pinned=pinned)

        # Page-locked staging: K/V stage slots, the Q block, host output slots.
        records = kv_record_pages(kv_source.kv_pages, kv_layout)
        record_bytes = max((token_scale_layout(r, kv_layout)[2] for r in records), default=4096)
        min_page = min((p.valid_tokens for p in kv_source.kv_pages), default=1)
        stage_count = 0
        if self.zero_copy_kv is None:
            stage_count = depth + math.ceil(plan.kv_chunk_tokens / max(1, min_page)) + 1
        q_bpt = q_layout.bytes_per_token
        max_q_page = max((p.valid_tokens for p in q_source.q_pages), default=1)
        n_out = 0 if (device_mode or self.direct_out is not None) else max(1, config.num_output_buffers)
        q_stage_needed = self.zero_copy_q is None
        available = memory_plan.available("pinned")
        slot_bytes = PinnedSlab(record_bytes, 0, pinned=False).slot_bytes
        # Shrink the stage ring to at most half of the pinned budget, then fit the Q rows.
        stage_count = min(stage_count, max(depth + 1, available // 2 // slot_bytes)) if stage_count else 0
        stage_bytes = stage_count * slot_bytes
        q_rows = plan.q_chunk_tokens
        per_row = q_bpt * ((1 if q_stage_needed else 0) + n_out)
        if per_row:
            fit = (available - stage_bytes) // per_row
            if n_out and fit < max_q_page:
                fit = (available - stage_bytes - n_out * max_q_page * q_bpt) // max(1, q_bpt * int(q_stage_needed))
            q_rows = min(q_rows, fit)
            if q_rows >= 256:
                q_rows -= q_rows % 256
        if q_rows < 1:
            raise MemoryError("pinned staging budget cannot hold one query block and the K/V stage ring")
        self.q_rows = q_rows
        out_rows = max(q_rows, max_q_page)
        total_pinned = stage_bytes + (q_rows * q_bpt if q_stage_needed else 0) + n_out * out_rows * q_bpt
        memory_plan.register("pinned", total_pinned)
        self.pinned_registered = total_pinned
        if stage_count:
            self.stages = _StageRing(record_bytes, stage_count, pinned)
        if q_stage_needed:
            self.q_stage = torch.empty((q_rows, q_layout.heads, q_layout.head_dim), dtype=q_layout.torch_dtype,
                                       pin_memory=pinned)
            if max_q_page > q_rows or any(p.valid_tokens > q_rows for p in q_source.q_pages):
                self.q_page_buffer = torch.empty((max_q_page, q_layout.heads, q_layout.head_dim),
                                                 dtype=q_layout.torch_dtype)
        self.out_stage = [torch.empty((out_rows, q_layout.heads, q_layout.head_dim), dtype=q_layout.torch_dtype,
                                      pin_memory=pinned) for _ in range(n_out)]
        self.out_futures = [[] for _ in range(n_out)]
        self.out_events = [None] * n_out
        self.pool = ThreadPoolExecutor(max_workers=max(1, config.io_workers), thread_name_prefix="seqattn-io")
        run_plan = replace(plan, q_chunk_tokens=q_rows) if q_rows < plan.q_chunk_tokens else plan
        with torch.cuda.device(device):
            self.workspace = CudaWorkspace(run_plan)
            if config.attention.enable_nvtx:
                self.workspace.enable_trace_ranges()
            if self.int8:
                # One fp16 scale per (row, K/V head) per ring slot, for K and for V.
                shape = (run_plan.kv_chunk_tokens, run_plan.kv_heads)
                ks = [torch.empty(shape, dtype=torch.float16, device=device) for _ in self.workspace.k]
                vs = [torch.empty(shape, dtype=torch.float16, device=device) for _ in self.workspace.k]
                self.scale_ring = ks + vs
                count = len(ks)
                _native.check(_native.lib().sa_pipeline_attach_int8_scales(
                    self.workspace.handle, (ctypes.c_void_p * count)(*[t.data_ptr() for t in ks]),
                    (ctypes.c_void_p * count)(*[t.data_ptr() for t in vs]), count),
                    "sa_pipeline_attach_int8_scales")
        self.q_event = torch.cuda.Event()
        self.q_event_pending = False

    # --- K/V pages -----------------------------------------------------------

    def submit_kv(self, runner, page: PageDescriptor, k0: int, issue, queue, stats) -> _Load:
        if self.zero_copy_kv is not None:
            k_rows, v_rows = self.zero_copy_kv.pinned_kv_rows(page.token_start, page.token_stop)
            self.cache.lookup(page)
            return _Load(page, None, k_rows.data_ptr(), v_rows.data_ptr(), None)
        slot, lookup = self.cache.lookup(page)
        stats.cache_lookup_seconds += lookup.seconds
        record = self.cache.record(page) if self.cache.records else None
        ks_offset, vs_offset, _ = token_scale_layout(record, self.kv_layout)
        if slot is not None:
            slab = self.cache.slab
            slab.hold(slot)
            base = slab.address(slot)
            return _Load(page, None, base, base + record.v_offset, ("cache", slot),
                         ks_address=base + ks_offset, vs_address=base + vs_offset)
        slot = self.cache.reserve(page)
        if slot is not None:
            slab = self.cache.slab
            slab.hold(slot)
            future = self.pool.submit(self._read_kv_into, slab, slot, page, record)
            base = slab.address(slot)
            return _Load(page, future, base, base + record.v_offset, ("cache", slot), commit_slot=slot,
                         ks_address=base + ks_offset, vs_address=base + vs_offset)
        # Uncached: a staging slot (flush queued rows if every slot is referenced).
        stages = self.stages
        while not stages.free:
            if not queue.rows:
                raise RuntimeError("K/V staging ring exhausted")
            issue(queue.rows)
        stage = stages.free.popleft()
        stages.slab.wait_reusable(stage)
        stages.slab.hold(stage)
        future = self.pool.submit(self._read_kv_into, stages.slab, stage, page, record)
        base = stages.slab.address(stage)
        return _Load(page, future, base, base + record.v_offset, ("stage", stage),
                     ks_address=base + ks_offset, vs_address=base + vs_offset)

    def _read_kv_into(self, slab: PinnedSlab, slot: int, page: PageDescriptor, record: PageDescriptor):
        """Read the page's record image into ``slot`` (I/O worker thread); INT8
        records then get their per-row scales."""
        destination = slab.bytes(slot)
        reader = self.kv_reader
        layout = self.kv_layout
        if hasattr(reader, "read_kv_record"):
            metrics = reader.read_kv_record(page, destination)
        else:
            dtype = layout.storage_torch_dtype
            shape = (record.padded_tokens, layout.heads, layout.head_dim)
            k_view = destination[: record.k_bytes].view(dtype).view(shape)
            v_view = destination[record.v_offset : record.v_offset + record.v_bytes].view(dtype).view(shape)
            scales = ()
            if self.int8:
                groups = record.scale_bytes // (2 * layout.heads)
                scales = tuple(
                    destination[offset : offset + record.scale_bytes].view(torch.float16).view(groups, layout.heads)
                    for offset in (record.k_scale_offset, record.v_scale_offset))
            metrics = reader.read_kv(page, k_view, v_view, *scales)
        if self.int8:
            expand_token_scales(destination, record, layout)
        return metrics

    def release(self, owner, event) -> None:
        if owner is None:
            return
        kind, slot = owner
        if kind == "cache":
            self.cache.slab.release(slot, event)
        else:
            self.stages.release(slot, event)

    # --- Q rows --------------------------------------------------------------

    def prefetch_q(self, block) -> None:
        """Start reading the next block's query pages into the Q staging
        buffer once the current block's Q copy has left it."""
        if self.zero_copy_q is not None:
            return
        self._submit_q_reads(block)

    def _submit_q_reads(self, block) -> None:
        if self.q_event_pending:
            self.q_event.synchronize()
            self.q_event_pending = False
        futures = []
        for piece in block.pieces:
            target = self.q_stage[piece.block_offset : piece.block_offset + piece.rows]
            futures.append(self.pool.submit(self._read_q_piece, piece, target))
        self.q_reads = (block, futures)

    def load_q_rows(self, runner, block, q_row_bytes, stats, global_start) -> int:
        stats.q_pages += sum(1 for piece in block.pieces if piece.page_offset == 0)
        if self.zero_copy_q is not None:
            return self.zero_copy_q.pinned_q_rows(global_start, global_start + block.rows).data_ptr()
        if self.q_reads is None or self.q_reads[0] is not block:
            self._submit_q_reads(block)
        futures = self.q_reads[1]
        self.q_reads = None
        wait_started = time.perf_counter()
        for future in futures:
            runner._account_read(stats, future.result(), self.q_is_nvme)
        stats.io_queue_wait_seconds += time.perf_counter() - wait_started
        return self.q_stage.data_ptr()

    def _read_q_piece(self, piece, target) -> PageReadMetrics:
        if piece.whole_page:
            return self.q_reader.read_q(piece.page, target)
        buffer = self.q_page_buffer
        metrics = self.q_reader.read_q(piece.page, buffer[: piece.page.valid_tokens])
        target.copy_(buffer[piece.page_offset : piece.page_offset + piece.rows])
        return metrics

    def q_loaded(self) -> None:
        if self.q_stage is not None:
            self.q_event.record(self.workspace.h2d_stream)
            self.q_event_pending = True

    # --- output --------------------------------------------------------------

    def next_device_slot(self) -> int:
        slot = self.device_slot % max(1, len(self.workspace.output))
        self.device_slot += 1
        return slot

    def wait_out_slot(self, slot: int, runner, stats) -> None:
        for future in self.out_futures[slot]:
            started = time.perf_counter()
            runner._account_write(stats, future.result(), self.out_is_nvme)
            stats.io_queue_wait_seconds += time.perf_counter() - started
        self.out_futures[slot] = []

    def write_group(self, runner, group: QGroup, slot: int, stats) -> None:
        """Hand the group's finished pages to the writer (after their D2H)."""
        event = torch.cuda.Event()
        event.record(self.workspace.d2h_stream)
        event.synchronize()
        data = self.out_stage[slot]
        offset = 0
        for page in group.pages:
            rows = data[offset : offset + page.valid_tokens]
            self.out_futures[slot].append(self.pool.submit(self.writer.write_page, page, rows))
            offset += page.valid_tokens

    def finish_writes(self, runner, stats) -> None:
        for slot in range(len(self.out_futures)):
            self.wait_out_slot(slot, runner, stats)

    # --- teardown ------------------------------------------------------------

    def abort(self) -> None:
        for futures in self.out_futures:
            for future in futures:
                future.cancel()
        if self.pool is not None:
            self.pool.shutdown(wait=True, cancel_futures=True)
            self.pool = None
        if self.writer is not None:
            self.writer.abort()
            self.writer = None

    def close(self) -> None:
        if self.pool is not None:
            self.pool.shutdown(wait=True, cancel_futures=True)
            self.pool = None
        if self.workspace is not None:
            torch.cuda.synchronize(self.workspace.device)
            self.workspace.close()
            self.workspace = None
        if self.cache is not None:
            self.cache.close()
        if self.kv_reader is not None:
            self.kv_reader.close()
        if self.q_reader is not None and self.q_reader is not self.kv_reader:
            self.q_reader.close()
        if self.stages is not None:
            self.stages.slab.close()
        self.q_stage = None
        self.out_stage = []
        self.scale_ring = []
        if self.pinned_registered:
            self.memory_plan.release("pinned", self.pinned_registered)
            self.pinned_registered = 0


__all__ = ["PagedAttentionRunner", "validate_source_contract"]
