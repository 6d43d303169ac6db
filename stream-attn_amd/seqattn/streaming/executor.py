"""Tensor-mode schedule (reference src/seqattn_core/streaming/executor.py:18-188).

Segment -> resident Q super-block -> K/V chunk loop.  Host output without a
consumer runs entirely inside the native pipeline (``sa_pipeline_run``: one
call, no per-chunk Python work).  Device consumers and device-resident outputs
drive the same pipeline one Q super-block at a time through its step API so a
Python callback can run between finalize and D2H.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable
from contextlib import nullcontext

import torch

from .. import _native
from ..stats import StreamingAttentionStats


def _bounds_array(bounds: list[int]) -> ctypes.Array:
    return (ctypes.c_int64 * len(bounds))(*bounds)


def _merge_stats(stats: StreamingAttentionStats, native: _native.PipelineStats) -> None:
    stats.h2d_bytes += native.h2d_bytes
    stats.d2h_bytes += native.d2h_bytes
    stats.q_chunks += native.q_chunks
    stats.kv_tiles += native.kv_tiles
    stats.max_resident_q_tokens = max(stats.max_resident_q_tokens, native.max_resident_q_tokens)


class HipExecutorMixin:
    def _range(self, name: str):
        if self.config.enable_nvtx:
            return torch.cuda.nvtx.range(name)
        return nullcontext()

    def _check_lse(self, lse: torch.Tensor | None, total_q: int) -> None:
        if lse is None:
            return
        if (
            lse.device.type != "cuda"
            or lse.dtype != torch.float32
            or lse.ndim != 2
            or lse.shape[0] != self.plan.q_heads
            or lse.shape[1] < total_q
            or lse.stride(1) != 1
        ):
            raise ValueError("lse_out must be a float32 device tensor [q_heads, >= total_q_tokens]")

    def _run_native(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        q_bounds: list[int],
        k_bounds: list[int],
        scale: float,
        causal: bool,
        out: torch.Tensor,
        stats: StreamingAttentionStats,
        lse: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Whole-run host output into a CPU ``out`` (one native call)."""
        workspace = self._workspace
        self._check_lse(lse, q_cpu.shape[0])
        native_stats = _native.PipelineStats()
        with torch.cuda.device(self.plan.device), self._range("seqattn:run"):
            status = _native.lib().sa_pipeline_run(
                workspace.handle,
                q_cpu.data_ptr(), k_cpu.data_ptr(), v_cpu.data_ptr(), out.data_ptr(),
                None if lse is None else lse.data_ptr(), 0 if lse is None else lse.stride(0),
                _bounds_array(q_bounds), _bounds_array(k_bounds), len(q_bounds) - 1,
                float(scale), int(bool(causal)),
                workspace.compute_stream.cuda_stream, ctypes.byref(native_stats),
            )
        _native.check(status, "sa_pipeline_run")
        _merge_stats(stats, native_stats)
        return out

    def _run_native_device_output(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        q_bounds: list[int],
        k_bounds: list[int],
        scale: float,
        causal: bool,
        out: torch.Tensor,
        stats: StreamingAttentionStats,
        lse: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Head-group schedule into a device ``out``: the unit launches write
        its rows directly (one native call, no output copy).  Ordered after
        the work the caller's current stream has enqueued so far, and the
        caller's stream waits for it in turn, as for HBM-resident inputs."""
        workspace = self._workspace
        self._check_lse(lse, q_cpu.shape[0])
        native_stats = _native.PipelineStats()
        compute = workspace.compute_stream
        with torch.cuda.device(self.plan.device):
            caller = torch.cuda.current_stream()
            if caller != compute:
                compute.wait_stream(caller)
        with torch.cuda.device(self.plan.device), self._range("seqattn:run"):
            status = _native.lib().sa_pipeline_run_device_output(
                workspace.handle,
                q_cpu.data_ptr(), k_cpu.data_ptr(), v_cpu.data_ptr(),
                out.data_ptr(), out.stride(0), out.stride(1),
                None if lse is None else lse.data_ptr(), 0 if lse is None else lse.stride(0),
                _bounds_array(q_bounds), _bounds_array(k_bounds), len(q_bounds) - 1,
                float(scale), int(bool(causal)),
                compute.cuda_stream, ctypes.byref(native_stats),
            )
        _native.check(status, "sa_pipeline_run_device_output")
        if caller != compute:
            caller.wait_stream(compute)
        _merge_stats(stats, native_stats)
        return out

    def _run_resident(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        q_bounds: list[int],
        k_bounds: list[int],
        scale: float,
        causal: bool,
        out: torch.Tensor,
        stats: StreamingAttentionStats,
        lse: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """HBM-resident inputs and output: one native call, no PCIe traffic.

        Enqueued on the runner's compute stream (torch's current stream at
        construction), ordered after the work the caller's current stream has
        enqueued so far, and the caller's stream waits for it in turn: the
        inputs may come from, and the output go to, work on any stream, and the
        caller synchronizes as with any torch op.
        """
        workspace = self._workspace
        self._check_lse(lse, q.shape[0])
        native_stats = _native.PipelineStats()
        compute = workspace.compute_stream
        with torch.cuda.device(self.plan.device):
            caller = torch.cuda.current_stream()
            longest_k = max((b - a for a, b in zip(k_bounds[:-1], k_bounds[1:])), default=0)
            stats.resident_scratch_bytes = workspace.attach_resident_scratch(
                longest_k, self.config.resident_scratch_limit_bytes
            )
            if caller != compute:
                compute.wait_stream(caller)
        with torch.cuda.device(self.plan.device), self._range("seqattn:run_resident"):
            status = _native.lib().sa_pipeline_run_resident(
                workspace.handle,
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                None if lse is None else lse.data_ptr(),
                q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                out.stride(0), out.stride(1), 0 if lse is None else lse.stride(0),
                _bounds_array(q_bounds), _bounds_array(k_bounds), len(q_bounds) - 1,
                float(scale), int(bool(causal)),
                compute.cuda_stream, ctypes.byref(native_stats),
            )
        _native.check(status, "sa_pipeline_run_resident")
        if caller != compute:
            caller.wait_stream(compute)
        _merge_stats(stats, native_stats)
        return out

    def _run_steps(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        q_bounds: list[int],
        k_bounds: list[int],
        scale: float,
        causal: bool,
        out: torch.Tensor,
        stats: StreamingAttentionStats,
        output_transform: Callable[[torch.Tensor, int, int], torch.Tensor] | None = None,
        lse: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Per-super-block schedule for consumers and device-resident outputs."""
        workspace = self._workspace
        plan = self.plan
        lib = _native.lib()
        handle = workspace.handle
        compute = workspace.compute_stream
        compute_ptr = compute.cuda_stream
        self._check_lse(lse, q_cpu.shape[0])
        native_stats = _native.PipelineStats()
        stats_ref = ctypes.byref(native_stats)
        q_row = q_cpu.shape[1] * q_cpu.shape[2] * q_cpu.element_size()
        kv_row = k_cpu.shape[1] * k_cpu.shape[2] * k_cpu.element_size()
        out_on_device = out.device.type == "cuda"
        reuse_q = output_transform is not None and plan.output_mode == "device_consumer"
        lse_ptr = None if lse is None else lse.data_ptr()
        lse_stride = 0 if lse is None else lse.stride(0)
        chunk_index = 0
        with torch.cuda.device(plan.device):
            for q_start, q_stop, k_start, k_stop in zip(
                q_bounds[:-1], q_bounds[1:], k_bounds[:-1], k_bounds[1:]
            ):
                causal_shift = (k_stop - k_start) - (q_stop - q_start)
                for q_tile_start in range(q_start, q_stop, plan.q_chunk_tokens):
                    q_tile_stop = min(q_tile_start + plan.q_chunk_tokens, q_stop)
                    n = q_tile_stop - q_tile_start
                    with self._range("seqattn:q_h2d"):
                        _native.check(
                            lib.sa_pipeline_load_q(
                                handle, q_cpu.data_ptr() + q_tile_start * q_row, n, compute_ptr, stats_ref
                            ),
                            "sa_pipeline_load_q",
                        )
                    with self._range("seqattn:fused_update"):
                        _native.check(
                            lib.sa_pipeline_stream_kv(
                                handle,
                                k_cpu.data_ptr() + k_start * kv_row,
                                v_cpu.data_ptr() + k_start * kv_row,
                                k_stop - k_start, n, q_tile_start - q_start, causal_shift,
                                float(scale), int(bool(causal)), compute_ptr, stats_ref,
                            ),
                            "sa_pipeline_stream_kv",
                        )
                    slot = chunk_index % plan.num_output_buffers
                    chunk_index += 1
                    if out_on_device and output_transform is None:
                        # Output stays in HBM: finalize straight into the caller's rows.
                        target = out[q_tile_start:q_tile_stop]
                        with self._range("seqattn:fused_finalize"):
                            _native.check(
                                lib.sa_pipeline_finalize_into(
                                    handle, target.data_ptr(), target.stride(0), target.stride(1), n,
                                    lse_ptr, lse_stride, q_tile_start, compute_ptr,
                                ),
                                "sa_pipeline_finalize_into",
                            )
                        continue
                    if reuse_q:
                        finalize_slot = -1
                        output_gpu = workspace.q[:n]
                    elif workspace.output:
                        finalize_slot = slot
                        output_gpu = workspace.output[slot][:n]
                    else:
                        finalize_slot = -1
                        output_gpu = workspace.q[:n]
                    with self._range("seqattn:fused_finalize"):
                        _native.check(
                            lib.sa_pipeline_finalize(
                                handle, finalize_slot, n, lse_ptr, lse_stride, q_tile_start, compute_ptr
                            ),
                            "sa_pipeline_finalize",
                        )
                    output_in_q = finalize_slot == -1
                    if output_transform is not None:
                        with self._range("seqattn:device_output_transform"), torch.cuda.stream(compute):
                            output_gpu = output_transform(output_gpu.reshape(n, -1), q_tile_start, q_tile_stop)
                            if output_gpu.device.type != "cuda":
                                raise ValueError("output_transform must return a CUDA tensor")
                            expected = out[q_tile_start:q_tile_stop].shape
                            if output_gpu.shape != expected:
                                raise ValueError(
                                    "output_transform result shape does not match the output slice: "
                                    f"{tuple(output_gpu.shape)} != {tuple(expected)}"
                                )
                            if output_gpu.dtype != out.dtype:
                                raise ValueError("output_transform result dtype must match out dtype")
                            if not output_gpu.is_contiguous():
                                output_gpu = output_gpu.contiguous()
                        aliases_q = (
                            output_gpu.untyped_storage().data_ptr()
                            == workspace.q.untyped_storage().data_ptr()
                        )
                        if output_in_q and not aliases_q:
                            _native.check(lib.sa_pipeline_release_q(handle, compute_ptr), "sa_pipeline_release_q")
                        output_in_q = output_in_q and aliases_q
                    destination = out[q_tile_start:q_tile_stop]
                    nbytes = output_gpu.numel() * output_gpu.element_size()
                    if out_on_device:
                        # Device consumer with a device-resident destination: a
                        # device-to-device copy on the compute stream.
                        with torch.cuda.stream(compute):
                            destination.copy_(output_gpu)
                        if output_in_q:
                            _native.check(lib.sa_pipeline_release_q(handle, compute_ptr), "sa_pipeline_release_q")
                        continue
                    with self._range("seqattn:output_d2h"):
                        _native.check(
                            lib.sa_pipeline_d2h(
                                handle, destination.data_ptr(), output_gpu.data_ptr(), nbytes, slot,
                                int(output_in_q), compute_ptr, stats_ref,
                            ),
                            "sa_pipeline_d2h",
                        )
                    output_gpu.record_stream(workspace.d2h_stream)
            if out_on_device:
                compute.synchronize()
            _native.check(lib.sa_pipeline_synchronize(handle), "sa_pipeline_synchronize")
        _merge_stats(stats, native_stats)
        return out


__all__ = ["HipExecutorMixin"]
