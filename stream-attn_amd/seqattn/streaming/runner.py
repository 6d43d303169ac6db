"""Reusable runner (reference src/seqattn_core/streaming/runner.py:18-179).

Same construction (``StreamingAttentionRunner(plan, config)``), call
signatures and validation as the reference.  Additive options:

* ``lse_out``: a float32 device tensor ``[q_heads, total_q_tokens]`` that
  receives the natural-log LSE of every query row; ``return_lse=True``
  allocates one and returns ``(out, lse)`` with the LSE copied to the host.
* ``out`` may be a device tensor: the output then stays in HBM (finalized
  straight into ``out``) and no D2H is issued.
* q, k and v may be device tensors on the plan's device (HBM-resident
  inputs): the same Q super-block / K/V chunk schedule then reads them in
  place, nothing crosses PCIe and the output is a device tensor.
* A plan of the head-group schedule (``schedule="head_groups"``) runs
  page-locked host inputs with one native call per run, each byte of Q, K
  and V crossing PCIe once, into a host ``out`` (a pageable one, with
  ``pin_output=False``, is written through 64 MiB of page-locked staging) or
  a device ``out`` (written by the launches, no output copy);
  ``run_with_device_output`` needs the default schedule.
"""

from __future__ import annotations

import time
from collections.abc import Callable

import torch

from ..config import StreamingAttentionConfig
from ..planner import AttentionPlan
from ..stats import StreamingAttentionStats
from ..validation import require_pinned_inputs, validate_device_qkv, validate_host_qkv
from .backend import resolve_backend
from .executor import HipExecutorMixin
from .workspace import CudaWorkspace


class StreamingAttentionRunner(HipExecutorMixin):
    """Reusable execution plan, device workspace and transfer pipeline.

    One runner is single-flight: create one runner per request stream when
    independent calls must execute concurrently.
    """

    def __init__(self, plan: AttentionPlan, config: StreamingAttentionConfig | None = None) -> None:
        self.plan = plan
        self.config = StreamingAttentionConfig() if config is None else config
        self.config.validate()
        if plan.output_mode != self.config.output_mode:
            raise ValueError("attention plan output_mode does not match runner config")
        self.backend = resolve_backend(self.config.backend, plan.dtype, plan.device, head_dim=plan.head_dim)
        self._workspace = CudaWorkspace(plan)
        if self.config.enable_nvtx:
            self._workspace.enable_trace_ranges()

    def close(self) -> None:
        """Release the pipeline's streams and events (buffers follow the runner)."""
        if self._workspace is not None:
            self._workspace.close()

    def release_resident_scratch(self) -> None:
        """Drop the transposed-V scratch that HBM-resident runs keep for the
        next run (as large as V; outside the planner's budget)."""
        if self._workspace is not None:
            self._workspace.release_resident_scratch()

    def _validate_inputs(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
    ) -> tuple[list[int], list[int]]:
        if q_cpu.device.type == "cuda":
            q_bounds, k_bounds = validate_device_qkv(
                q_cpu, k_cpu, v_cpu, cu_seqlens_q, cu_seqlens_k, self._device()
            )
        else:
            q_bounds, k_bounds = validate_host_qkv(q_cpu, k_cpu, v_cpu, cu_seqlens_q, cu_seqlens_k)
        if q_cpu.shape[1:] != (self.plan.q_heads, self.plan.head_dim):
            raise ValueError("q shape does not match the runner plan")
        if k_cpu.shape[1:] != (self.plan.kv_heads, self.plan.head_dim):
            raise ValueError("k/v shape does not match the runner plan")
        if q_cpu.dtype != self.plan.dtype:
            raise ValueError("input dtype does not match the runner plan")
        if q_cpu.shape[0] > self.plan.max_q_tokens or k_cpu.shape[0] > self.plan.max_kv_tokens:
            raise ValueError("input token count exceeds the runner plan")
        return q_bounds, k_bounds

    def _device(self) -> torch.device:
        device = self.plan.device
        return device if device.index is not None else torch.device("cuda", torch.cuda.current_device())

    def _prepare_io(self, q_cpu, k_cpu, v_cpu, out: torch.Tensor) -> None:
        if self.config.require_pinned:
            require_pinned_inputs(q_cpu, k_cpu, v_cpu)
        if out.device.type == "cpu" and self.config.pin_output and not out.is_pinned():
            raise ValueError("asynchronous D2H requires a pinned out tensor")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")

    def _prepare_stats(self, stats: StreamingAttentionStats | None) -> StreamingAttentionStats:
        stats = StreamingAttentionStats() if stats is None else stats
        stats.backend = self.backend
        stats.estimated_workspace_bytes = self.plan.estimated_workspace_bytes
        stats.q_chunk_tokens = self.plan.q_chunk_tokens
        stats.kv_chunk_tokens = self.plan.kv_chunk_tokens
        return stats

    def _lse_buffer(self, total_q: int, lse_out: torch.Tensor | None, return_lse: bool):
        if lse_out is not None or not return_lse:
            return lse_out
        return torch.empty((self.plan.q_heads, total_q), dtype=torch.float32, device=self.plan.device)

    @torch.inference_mode()
    def __call__(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        *,
        softmax_scale: float | None = None,
        causal: bool = False,
        out: torch.Tensor | None = None,
        stats: StreamingAttentionStats | None = None,
        lse_out: torch.Tensor | None = None,
        return_lse: bool = False,
    ):
        q_bounds, k_bounds = self._validate_inputs(q_cpu, k_cpu, v_cpu, cu_seqlens_q, cu_seqlens_k)
        if self.plan.output_mode == "device_consumer":
            raise ValueError("a device_consumer runner requires run_with_device_output()")
        scale = self.plan.head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
        if q_cpu.device.type == "cuda":
            return self._call_resident(
                q_cpu, k_cpu, v_cpu, q_bounds, k_bounds, scale, causal, out, stats, lse_out, return_lse
            )
        if out is None:
            out = torch.empty(
                q_cpu.shape, dtype=q_cpu.dtype, device="cpu",
                pin_memory=self.config.pin_output and torch.cuda.is_available(),
            )
        if out.shape != q_cpu.shape or out.dtype != q_cpu.dtype or out.device.type not in {"cpu", "cuda"}:
            raise ValueError("out must be a CPU tensor matching q shape and dtype")
        self._prepare_io(q_cpu, k_cpu, v_cpu, out)
        if self.plan.schedule == "head_groups":
            if out.device.type != "cpu" and (out.device != self._device() or out.stride(2) != 1):
                raise ValueError("a device out must be on the plan's device with unit stride over head_dim")
            if not all(t.is_pinned() for t in (q_cpu, k_cpu, v_cpu)):
                # Strided copies between pageable memory and the device are
                # staged by the runtime row by row.
                raise ValueError("schedule='head_groups' copies head columns with strided copies, which need "
                                 "page-locked q, k and v")
            # A pageable out (pin_output=False) is written through page-locked
            # staging by the pipeline.
            self._workspace.stage_output(out.device.type == "cpu" and not out.is_pinned())
        lse = self._lse_buffer(q_cpu.shape[0], lse_out, return_lse)
        stats = self._prepare_stats(stats)
        started = time.perf_counter()
        if out.device.type == "cpu":
            result = self._run_native(q_cpu, k_cpu, v_cpu, q_bounds, k_bounds, scale, causal, out, stats, lse)
        elif self.plan.schedule == "head_groups":
            result = self._run_native_device_output(q_cpu, k_cpu, v_cpu, q_bounds, k_bounds, scale, causal, out,
                                                    stats, lse)
        else:
            result = self._run_steps(q_cpu, k_cpu, v_cpu, q_bounds, k_bounds, scale, causal, out, stats, lse=lse)
        stats.wall_seconds += time.perf_counter() - started
        if return_lse:
            return result, lse.cpu() if lse_out is None else lse
        return result

    def _call_resident(self, q, k, v, q_bounds, k_bounds, scale, causal, out, stats, lse_out, return_lse):
        if out is None:
            out = torch.empty_like(q)
        if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
            raise ValueError("out must be a device tensor matching q shape and dtype")
        if out.stride(2) != 1 or any(t.stride(2) != 1 for t in (q, k, v)):
            raise ValueError("device-resident tensors need unit stride over head_dim")
        lse = self._lse_buffer(q.shape[0], lse_out, return_lse)
        stats = self._prepare_stats(stats)
        started = time.perf_counter()
        result = self._run_resident(q, k, v, q_bounds, k_bounds, scale, causal, out, stats, lse)
        stats.wall_seconds += time.perf_counter() - started
        if return_lse:
            return result, lse
        return result

    @torch.inference_mode()
    def run_with_device_output(
        self,
        q_cpu: torch.Tensor,
        k_cpu: torch.Tensor,
        v_cpu: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        *,
        output_transform: Callable[[torch.Tensor, int, int], torch.Tensor] | None,
        out: torch.Tensor,
        softmax_scale: float | None = None,
        causal: bool = False,
        stats: StreamingAttentionStats | None = None,
        lse_out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Consume each finalized device tile before it leaves HBM.

        ``output_transform(tile [q_tokens, heads*head_dim], start, stop)`` runs
        on the compute stream and returns the tensor copied into
        ``out[start:stop]``.  ``out`` may be a CPU tensor (D2H, as the
        reference) or a device tensor (the result stays in HBM).
        """
        if q_cpu.device.type != "cpu":
            raise ValueError("seqattn expects CPU-backed q, k, and v tensors")
        if self.plan.schedule == "head_groups":
            raise ValueError("run_with_device_output needs a Q-block plan (schedule='q_blocks', or "
                             "output_mode='device_consumer' with schedule='auto'): head groups finish every "
                             "query row of a head group at once, not tile by tile")
        q_bounds, k_bounds = self._validate_inputs(q_cpu, k_cpu, v_cpu, cu_seqlens_q, cu_seqlens_k)
        if out.device.type not in {"cpu", "cuda"} or out.shape[0] != q_cpu.shape[0]:
            raise ValueError("out must be a CPU tensor with one row per query token")
        self._prepare_io(q_cpu, k_cpu, v_cpu, out)
        scale = self.plan.head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
        stats = self._prepare_stats(stats)
        started = time.perf_counter()
        result = self._run_steps(
            q_cpu, k_cpu, v_cpu, q_bounds, k_bounds, scale, causal, out, stats,
            output_transform=output_transform, lse=lse_out,
        )
        stats.wall_seconds += time.perf_counter() - started
        return result


__all__ = ["StreamingAttentionRunner"]
