"""Hidden states -> QKV projection -> streamed attention -> output projection
(reference src/seqattn_core/projection/runner.py:16-259).

Same construction (``ProjectedAttentionRunner(plan, attention_config,
pipeline_config)``), call signature, stats and validation messages as the
reference.  The pipeline has two phases, because exact self-attention needs
every K/V row before any query row can finish:

1. **Projection producer** (``project_qkv_to_host``): the pinned hidden rows
   cross PCIe in ``projection_chunk_tokens`` tiles on an H2D stream, the
   caller's ``project_qkv`` runs on the compute stream, and the projected
   Q/K/V tiles go back to pinned host buffers on a D2H stream.  Up to
   ``num_projection_buffers`` tiles are in flight.
2. **Attention + output projection** (``run_with_device_output`` of the
   streamed runner): each finalized attention tile is handed to
   ``output_projector`` while still in HBM and only the projected rows are
   copied out, so no raw attention output ever reaches host memory.

``qkv_residency="hbm"`` (additive) keeps phase 1's Q/K/V in device memory
instead.  Phase 2 then runs the streamed schedule on the resident Q/K/V and
finalizes each Q block into the rows of Q it has just consumed (a block's Q
rows are read only by its own launches, which precede its finalize on the
compute stream).  The output projection follows tile by tile with the D2H
of each projected tile overlapping the next tile's projection.  Q/K/V never
cross PCIe; the device holds ``2 * tokens * (q_heads + kv_heads) * head_dim``
bytes of Q/K/V more than in host residency.
"""

from __future__ import annotations

import time
from contextlib import nullcontext
from dataclasses import replace

import torch

from ..config import ProjectionPipelineConfig, StreamingAttentionConfig
from ..planner import AttentionPlan, build_plan
from ..stats import ProjectedAttentionStats
from ..streaming import StreamingAttentionRunner
from .types import OutputProjector, QKVProjector
from .workspace import ProjectionWorkspace


class ProjectedAttentionRunner:
    """Reusable CPU-hidden -> QKV -> attention -> output-projection pipeline."""

    def __init__(
        self,
        plan: AttentionPlan,
        attention_config: StreamingAttentionConfig | None = None,
        pipeline_config: ProjectionPipelineConfig | None = None,
    ) -> None:
        self.attention_config = StreamingAttentionConfig() if attention_config is None else attention_config
        self.pipeline_config = ProjectionPipelineConfig() if pipeline_config is None else pipeline_config
        self.attention_config.validate()
        self.pipeline_config.validate()
        if self.attention_config.schedule == "head_groups":
            raise ValueError("the projected pipeline projects each finished Q tile: it needs schedule='q_blocks'")
        # "auto" plans Q blocks here: the output projection consumes Q tiles.
        self.attention_config = replace(self.attention_config, schedule="q_blocks")
        # The plan is rebuilt against the runner's own attention config, as
        # the reference does, so a plan made with other launch settings
        # still gets a consistent workspace.
        self.plan = build_plan(
            q_heads=plan.q_heads,
            kv_heads=plan.kv_heads,
            head_dim=plan.head_dim,
            dtype=plan.dtype,
            device=plan.device,
            max_q_tokens=plan.max_q_tokens,
            max_kv_tokens=plan.max_kv_tokens,
            config=self.attention_config,
        )
        plan = self.plan
        if plan.device.type != "cuda":
            raise ValueError("the projected pipeline requires a CUDA device")
        if self.attention_config.backend not in {"auto", "hip", "triton"}:
            raise ValueError("the projected pipeline requires the native attention backend")
        self.hbm_resident = self.pipeline_config.qkv_residency == "hbm"
        if (
            not self.hbm_resident
            and self.attention_config.require_pinned
            and not self.pipeline_config.pin_qkv
        ):
            raise ValueError("streamed attention requires pinned Q/K/V backing buffers")

        self.attention = StreamingAttentionRunner(plan, self.attention_config)
        self.q_cpu: torch.Tensor | None = None
        self.k_cpu: torch.Tensor | None = None
        self.v_cpu: torch.Tensor | None = None
        self.q_device: torch.Tensor | None = None
        self.k_device: torch.Tensor | None = None
        self.v_device: torch.Tensor | None = None
        if self.hbm_resident:
            self._allocate_device_qkv()
        else:
            self._allocate_host_qkv()
        self._projection_workspace: ProjectionWorkspace | None = None

    # -- buffers -------------------------------------------------------------

    def _qkv_shapes(self):
        plan = self.plan
        return (
            (plan.max_q_tokens, plan.q_heads, plan.head_dim),
            (plan.max_kv_tokens, plan.kv_heads, plan.head_dim),
        )

    def _allocate_host_qkv(self) -> None:
        q_shape, kv_shape = self._qkv_shapes()
        pin = self.pipeline_config.pin_qkv
        self.q_cpu = torch.empty(q_shape, dtype=self.plan.dtype, device="cpu", pin_memory=pin)
        self.k_cpu = torch.empty(kv_shape, dtype=self.plan.dtype, device="cpu", pin_memory=pin)
        self.v_cpu = torch.empty(kv_shape, dtype=self.plan.dtype, device="cpu", pin_memory=pin)

    def _allocate_device_qkv(self) -> None:
        q_shape, kv_shape = self._qkv_shapes()
        device = self.attention._device()
        self.q_device = torch.empty(q_shape, dtype=self.plan.dtype, device=device)
        self.k_device = torch.empty(kv_shape, dtype=self.plan.dtype, device=device)
        self.v_device = torch.empty(kv_shape, dtype=self.plan.dtype, device=device)

    def _range(self, name: str):
        if self.pipeline_config.enable_nvtx:
            return torch.cuda.nvtx.range(name)
        return nullcontext()

    def _workspace_for(self, hidden_features: int) -> ProjectionWorkspace:
        if self._projection_workspace is None:
            self._projection_workspace = ProjectionWorkspace(
                hidden_features=hidden_features,
                dtype=self.plan.dtype,
                device=self.attention._device(),
                config=self.pipeline_config,
            )
        elif self._projection_workspace.hidden_features != hidden_features:
            raise ValueError("hidden feature size changed for a persistent ProjectedAttentionRunner")
        return self._projection_workspace

    # -- validation ----------------------------------------------------------

    def _validate_hidden(self, hidden_cpu: torch.Tensor) -> None:
        if hidden_cpu.device.type != "cpu" or hidden_cpu.ndim != 2:
            raise ValueError("hidden_cpu must use CPU [tokens, hidden_features] layout")
        if not hidden_cpu.is_contiguous():
            raise ValueError("hidden_cpu must be contiguous")
        if hidden_cpu.dtype != self.plan.dtype:
            raise ValueError("hidden_cpu dtype must match the attention plan")
        if self.pipeline_config.require_pinned_hidden and not hidden_cpu.is_pinned():
            raise ValueError("asynchronous projection requires pinned hidden_cpu")
        tokens = hidden_cpu.shape[0]
        if tokens > self.plan.max_q_tokens or tokens > self.plan.max_kv_tokens:
            raise ValueError("hidden token count exceeds the runner plan")

    def _validate_projected_tile(self, q, k, v, tokens: int) -> None:
        expected_q = (tokens, self.plan.q_heads, self.plan.head_dim)
        expected_kv = (tokens, self.plan.kv_heads, self.plan.head_dim)
        if q.shape != expected_q:
            raise ValueError(f"project_qkv returned q shape {tuple(q.shape)}, expected {expected_q}")
        if k.shape != expected_kv or v.shape != expected_kv:
            raise ValueError(
                "project_qkv returned invalid k/v shapes: "
                f"{tuple(k.shape)}, {tuple(v.shape)}, expected {expected_kv}"
            )
        device = self.attention._device()
        if any(t.device != device for t in (q, k, v)):
            raise ValueError("project_qkv must return tensors on the planned CUDA device")
        if any(t.dtype != self.plan.dtype for t in (q, k, v)):
            raise ValueError("project_qkv output dtype must match the attention plan")

    def _validate_out(self, out: torch.Tensor | None, tokens: int, output_features: int | None) -> torch.Tensor:
        if out is None:
            if output_features is None or output_features <= 0:
                raise ValueError("output_features must be positive when out is omitted")
            out = torch.empty(
                (tokens, output_features), dtype=self.plan.dtype, device="cpu",
                pin_memory=self.pipeline_config.pin_output,
            )
        if out.device.type != "cpu" or out.ndim != 2 or out.shape[0] != tokens:
            raise ValueError("out must use CPU [tokens, output_features] layout")
        if out.dtype != self.plan.dtype:
            raise ValueError("out dtype must match the attention plan")
        if self.pipeline_config.pin_output and not out.is_pinned():
            raise ValueError("asynchronous output D2H requires pinned out")
        return out

    # -- phase 1: projection producer ------------------------------------------

    def _project(self, hidden_cpu, project_qkv, stats, q_dst, k_dst, v_dst) -> None:
        """Chunked hidden H2D -> project_qkv -> copy into ``q/k/v_dst`` rows.

        Host destinations are written on the D2H stream; device destinations
        on the compute stream right behind the projection.
        """
        workspace = self._workspace_for(hidden_cpu.shape[1])
        to_host = q_dst.device.type == "cpu"
        try:
            self._project_chunks(hidden_cpu, project_qkv, stats, q_dst, k_dst, v_dst, workspace, to_host)
        finally:
            # Also on a failed callback: no copy or projection of this call
            # may still touch the hidden slots when the next call refills them.
            workspace.drain()

    def _project_chunks(self, hidden_cpu, project_qkv, stats, q_dst, k_dst, v_dst, workspace, to_host) -> None:
        tokens, hidden_features = hidden_cpu.shape
        chunk = self.pipeline_config.projection_chunk_tokens
        pinned_hidden = hidden_cpu.is_pinned()
        element = hidden_cpu.element_size()
        for chunk_index, start in enumerate(range(0, tokens, chunk)):
            stop = min(start + chunk, tokens)
            n = stop - start
            slot = chunk_index % len(workspace.hidden)
            workspace.reclaim(slot)
            with self._range("seqattn:projection_hidden_h2d"), torch.cuda.stream(workspace.h2d_stream):
                workspace.hidden[slot][:n].copy_(hidden_cpu[start:stop], non_blocking=pinned_hidden)
                workspace.input_ready[slot].record(workspace.h2d_stream)
            with torch.cuda.stream(workspace.compute_stream):
                workspace.compute_stream.wait_event(workspace.input_ready[slot])
                with self._range("seqattn:qkv_projection"):
                    q, k, v = project_qkv(workspace.hidden[slot][:n], start, stop)
                    self._validate_projected_tile(q, k, v, n)
                workspace.projected_ready[slot].record(workspace.compute_stream)
                if not to_host:
                    q_dst[start:stop].copy_(q)
                    k_dst[start:stop].copy_(k)
                    v_dst[start:stop].copy_(v)
                    workspace.copy_done[slot].record(workspace.compute_stream)
            if to_host:
                with self._range("seqattn:projection_qkv_d2h"), torch.cuda.stream(workspace.d2h_stream):
                    workspace.d2h_stream.wait_event(workspace.projected_ready[slot])
                    q_dst[start:stop].copy_(q, non_blocking=q_dst.is_pinned())
                    k_dst[start:stop].copy_(k, non_blocking=k_dst.is_pinned())
                    v_dst[start:stop].copy_(v, non_blocking=v_dst.is_pinned())
                    workspace.copy_done[slot].record(workspace.d2h_stream)
                stats.projection_qkv_d2h_bytes += sum(t.numel() * t.element_size() for t in (q, k, v))
            workspace.keepalive[slot] = (q, k, v)
            workspace.busy[slot] = True
            stats.projection_chunks += 1
            stats.projection_hidden_h2d_bytes += n * hidden_features * element

    def project_qkv_to_host(
        self,
        hidden_cpu: torch.Tensor,
        project_qkv: QKVProjector,
        stats: ProjectedAttentionStats | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Run the chunked projection producer and return CPU-backed Q/K/V views."""
        stats = ProjectedAttentionStats() if stats is None else stats
        self._validate_hidden(hidden_cpu)
        stats.backend = self.attention.backend
        if self.q_cpu is None:
            self._allocate_host_qkv()
        tokens = hidden_cpu.shape[0]
        torch.cuda.synchronize(self.plan.device)
        started = time.perf_counter()
        self._project(hidden_cpu, project_qkv, stats, self.q_cpu, self.k_cpu, self.v_cpu)
        stats.projection_seconds += time.perf_counter() - started
        views = (self.q_cpu[:tokens], self.k_cpu[:tokens], self.v_cpu[:tokens])
        stats.qkv_host_bytes = sum(t.numel() * t.element_size() for t in views)
        return views

    def project_qkv_to_device(
        self,
        hidden_cpu: torch.Tensor,
        project_qkv: QKVProjector,
        stats: ProjectedAttentionStats | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The producer phase with device-resident results (additive).

        Returns views of the runner's device Q/K/V buffers; they stay valid
        until the next call on this runner.
        """
        stats = ProjectedAttentionStats() if stats is None else stats
        self._validate_hidden(hidden_cpu)
        stats.backend = self.attention.backend
        if self.q_device is None:
            self._allocate_device_qkv()
        tokens = hidden_cpu.shape[0]
        torch.cuda.synchronize(self.plan.device)
        started = time.perf_counter()
        self._project(hidden_cpu, project_qkv, stats, self.q_device, self.k_device, self.v_device)
        stats.projection_seconds += time.perf_counter() - started
        return self.q_device[:tokens], self.k_device[:tokens], self.v_device[:tokens]

    # -- phase 2 ---------------------------------------------------------------

    @torch.inference_mode()
    def __call__(
        self,
        hidden_cpu: torch.Tensor,
        cu_seqlens: torch.Tensor,
        *,
        project_qkv: QKVProjector,
        output_projector: OutputProjector,
        output_features: int | None = None,
        out: torch.Tensor | None = None,
        softmax_scale: float | None = None,
        causal: bool = False,
        stats: ProjectedAttentionStats | None = None,
    ) -> torch.Tensor:
        self._validate_hidden(hidden_cpu)
        tokens = hidden_cpu.shape[0]
        out = self._validate_out(out, tokens, output_features)
        stats = ProjectedAttentionStats() if stats is None else stats
        stats.backend = self.attention.backend
        started = time.perf_counter()
        raw_output_bytes = tokens * self.plan.q_heads * self.plan.head_dim * out.element_size()
        if self.hbm_resident:
            q, k, v = self.project_qkv_to_device(hidden_cpu, project_qkv, stats)
            stats.raw_attention_roundtrip_bytes_avoided += 2 * raw_output_bytes
            attention_started = time.perf_counter()
            self._attend_resident(q, k, v, cu_seqlens, output_projector, out, softmax_scale, causal, stats)
        else:
            q, k, v = self.project_qkv_to_host(hidden_cpu, project_qkv, stats)
            stats.raw_attention_roundtrip_bytes_avoided += 2 * raw_output_bytes
            attention_started = time.perf_counter()
            self.attention.run_with_device_output(
                q, k, v, cu_seqlens, cu_seqlens,
                output_transform=output_projector, out=out,
                softmax_scale=softmax_scale, causal=causal, stats=stats.attention,
            )
        stats.attention_output_seconds += time.perf_counter() - attention_started
        stats.wall_seconds += time.perf_counter() - started
        return out

    def _attend_resident(self, q, k, v, cu_seqlens, output_projector, out, softmax_scale, causal, stats) -> None:
        """Resident attention finalized into ``q``, then the output projection
        tile by tile (segment-bounded Q-chunk tiles, as the streamed runner
        hands them out) with each projected tile's D2H overlapping the next
        tile's projection."""
        attention = self.attention
        attention_stats = attention._prepare_stats(stats.attention)
        q_bounds, k_bounds = attention._validate_inputs(q, k, v, cu_seqlens, cu_seqlens)
        scale = self.plan.head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
        run_started = time.perf_counter()
        attention._run_resident(q, k, v, q_bounds, k_bounds, scale, causal, q, attention_stats)

        workspace = self._projection_workspace
        compute = attention._workspace.compute_stream
        d2h = workspace.d2h_stream
        ready = [torch.cuda.Event(), torch.cuda.Event()]
        done = [torch.cuda.Event(), torch.cuda.Event()]
        held: list[torch.Tensor | None] = [None, None]
        chunk = self.plan.q_chunk_tokens
        tiles = [
            (tile, min(tile + chunk, segment_stop))
            for segment_start, segment_stop in zip(q_bounds[:-1], q_bounds[1:])
            for tile in range(segment_start, segment_stop, chunk)
        ]
        for index, (start, stop) in enumerate(tiles):
            slot = index % 2
            if held[slot] is not None:
                done[slot].synchronize()
                held[slot] = None
            with self._range("seqattn:device_output_transform"), torch.cuda.stream(compute):
                projected = output_projector(q[start:stop].reshape(stop - start, -1), start, stop)
                if projected.device.type != "cuda":
                    raise ValueError("output_transform must return a CUDA tensor")
                expected = out[start:stop].shape
                if projected.shape != expected:
                    raise ValueError(
                        "output_transform result shape does not match the output slice: "
                        f"{tuple(projected.shape)} != {tuple(expected)}"
                    )
                if projected.dtype != out.dtype:
                    raise ValueError("output_transform result dtype must match out dtype")
                projected = projected.contiguous()
                ready[slot].record(compute)
            with self._range("seqattn:output_d2h"), torch.cuda.stream(d2h):
                d2h.wait_event(ready[slot])
                out[start:stop].copy_(projected, non_blocking=out.is_pinned())
                done[slot].record(d2h)
            held[slot] = projected
            attention_stats.d2h_bytes += projected.numel() * projected.element_size()
        d2h.synchronize()
        attention_stats.wall_seconds += time.perf_counter() - run_started


__all__ = ["ProjectedAttentionRunner"]
