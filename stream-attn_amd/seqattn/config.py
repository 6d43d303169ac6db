"""Execution policies (reference src/seqattn_core/config.py:6-142).

Field names, defaults and validation messages follow the reference so callers
and configuration files carry over unchanged.  Differences:

* ``backend`` additionally accepts ``"hip"``, the native gfx950 backend.
  ``"triton"`` is accepted as an alias of ``"hip"`` so existing call sites run
  unchanged; no Triton code exists in this package.
* ``output_mode`` additionally accepts ``"host_aliased"``: host output that is
  finalized into the resident Q buffer and copied back from there, which frees
  the raw output slots from the HBM budget (a larger resident Q block and
  fewer passes over K/V).
* ``schedule`` selects how the workspace is filled.  ``"q_blocks"`` (the
  default) is the reference's schedule: a resident Q super-block spans every
  head of a token range and all of K/V streams through the ring once per
  block.  ``"head_groups"`` keeps every token of a group of K/V heads (with
  their query heads) in HBM at once, so each byte of Q, K and V crosses PCIe
  once per run; it writes a host or a device output but no device consumer,
  and its results equal the default schedule's bit for bit.  ``"auto"``
  plans head groups when they fit the budget, the output is not a device
  consumer's and ``require_pinned`` holds, and Q blocks otherwise.
"""

from __future__ import annotations

from dataclasses import dataclass, field

BACKENDS = {"auto", "hip", "triton", "reference"}
OUTPUT_MODES = {"host", "host_aliased", "device_consumer"}
SCHEDULES = {"q_blocks", "head_groups", "auto"}


@dataclass(frozen=True)
class StreamingAttentionConfig:
    """Execution policy for CPU-backed exact attention.

    ``workspace_budget_bytes`` covers operator-owned device buffers only
    (resident Q, FP32 state, raw output slots, K/V ring); the HIP context and
    caller-owned allocations are outside it.
    """

    workspace_budget_bytes: int | None = None
    q_chunk_tokens: int | None = None
    kv_chunk_tokens: int | None = None
    num_kv_buffers: int = 2
    num_output_buffers: int = 1
    output_mode: str = "host"
    # Leaving all launch parameters unset selects the device/shape preset;
    # setting any one switches to the portable 64x64/4/2 baseline with the
    # supplied values as overrides.  block_m / block_n set the alignment of the
    # planned Q and K/V chunks; the gfx950 kernel's own tile geometry is fixed
    # (64 keys per tile; 384 queries per workgroup for head_dim 72-128, 256
    # for head_dim <= 64 and 128 for head_dim 256; K/V tiles double-buffered
    # in LDS).
    block_m: int | None = None
    block_n: int | None = None
    num_warps: int | None = None
    num_stages: int | None = None
    backend: str = "auto"
    require_pinned: bool = True
    pin_output: bool = True
    enable_nvtx: bool = False
    # HBM-resident inputs with head_dim 128 read V through a transposed copy
    # in device scratch (kv_heads * 128 * kv_tokens * 2 bytes, outside the
    # workspace budget).  None: no cap; 0: never; otherwise the largest
    # scratch the runner may allocate.  Without it V is read in place, with
    # bit-identical results.
    resident_scratch_limit_bytes: int | None = None
    # "q_blocks": the reference's Q super-block schedule.  "head_groups":
    # every token of a group of K/V heads resident at once (Q, K and V cross
    # PCIe once; no device consumer).  "auto": head groups when they fit
    # (with require_pinned and no device consumer), else Q blocks.
    schedule: str = "q_blocks"

    def validate(self) -> None:
        if self.workspace_budget_bytes is not None and self.workspace_budget_bytes <= 0:
            raise ValueError("workspace_budget_bytes must be positive")
        if self.resident_scratch_limit_bytes is not None and self.resident_scratch_limit_bytes < 0:
            raise ValueError("resident_scratch_limit_bytes must be non-negative")
        if self.q_chunk_tokens is not None and self.q_chunk_tokens <= 0:
            raise ValueError("q_chunk_tokens must be positive")
        if self.kv_chunk_tokens is not None and self.kv_chunk_tokens <= 0:
            raise ValueError("kv_chunk_tokens must be positive")
        if self.num_kv_buffers not in {1, 2, 3}:
            raise ValueError("num_kv_buffers must be 1, 2, or 3")
        if self.num_output_buffers not in {1, 2}:
            raise ValueError("num_output_buffers must be 1 or 2")
        if self.output_mode not in OUTPUT_MODES:
            raise ValueError("output_mode must be 'host', 'host_aliased' or 'device_consumer'")
        if self.block_m is not None and self.block_m not in {16, 32, 64, 128}:
            raise ValueError("block_m must be one of 16, 32, 64, 128")
        if self.block_n is not None and self.block_n not in {16, 32, 64, 128}:
            raise ValueError("block_n must be one of 16, 32, 64, 128")
        if self.num_warps is not None and self.num_warps not in {2, 4, 8}:
            raise ValueError("num_warps must be 2, 4, or 8")
        if self.num_stages is not None and self.num_stages not in {1, 2, 3, 4}:
            raise ValueError("num_stages must be within [1, 4]")
        if self.backend not in BACKENDS:
            raise ValueError(f"unsupported backend: {self.backend}")
        if self.schedule not in SCHEDULES:
            raise ValueError("schedule must be 'q_blocks', 'head_groups' or 'auto'")
        if self.schedule == "head_groups" and self.output_mode == "device_consumer":
            raise ValueError("schedule='head_groups' writes a host or device output but has no "
                             "device consumer; device_consumer output needs schedule='q_blocks'")


@dataclass(frozen=True)
class PagedAttentionConfig:
    """Execution and memory policy for paged CPU/NVMe attention.

    The host budget covers allocations owned by the operator.  Caller-owned
    tensors passed through ``MemoryPageSource`` are excluded.
    """

    attention: StreamingAttentionConfig = field(
        default_factory=lambda: StreamingAttentionConfig(
            workspace_budget_bytes=2 * 2**30,
            output_mode="host",
        )
    )
    host_memory_budget_bytes: int = 8 * 2**30
    pinned_staging_budget_bytes: int = 1 * 2**30
    direct_io_bounce_budget_bytes: int = 512 * 2**20
    metadata_margin_bytes: int = 128 * 2**20
    page_target_bytes: int = 16 * 2**20
    io_workers: int = 4
    io_queue_depth: int = 4
    num_output_buffers: int = 2
    cache_hot_fraction: float = 0.8
    direct_io: bool = True
    kv_storage_dtype: str = "bf16"
    quant_group_tokens: int = 64

    def validate(self) -> None:
        self.attention.validate()
        if self.host_memory_budget_bytes <= 0:
            raise ValueError("host_memory_budget_bytes must be positive")
        for name, value in (
            ("pinned_staging_budget_bytes", self.pinned_staging_budget_bytes),
            ("direct_io_bounce_budget_bytes", self.direct_io_bounce_budget_bytes),
            ("metadata_margin_bytes", self.metadata_margin_bytes),
        ):
            if value < 0:
                raise ValueError(f"{name} must be non-negative")
        reserved = (
            self.pinned_staging_budget_bytes
            + self.direct_io_bounce_budget_bytes
            + self.metadata_margin_bytes
        )
        if reserved >= self.host_memory_budget_bytes:
            raise ValueError(
                "pinned, bounce, and metadata reservations must leave room for the DRAM cache"
            )
        if self.page_target_bytes <= 0:
            raise ValueError("page_target_bytes must be positive")
        if self.io_workers <= 0:
            raise ValueError("io_workers must be positive")
        if self.io_queue_depth <= 0:
            raise ValueError("io_queue_depth must be positive")
        if self.num_output_buffers not in {1, 2}:
            raise ValueError("num_output_buffers must be 1 or 2")
        if not 0.0 <= self.cache_hot_fraction <= 1.0:
            raise ValueError("cache_hot_fraction must be within [0, 1]")
        if self.kv_storage_dtype not in {"bf16", "fp16", "fp32", "int8"}:
            raise ValueError("kv_storage_dtype must be bf16, fp16, fp32, or int8")
        if self.quant_group_tokens != 64:
            raise ValueError("V1 INT8 storage requires quant_group_tokens=64")


QKV_RESIDENCIES = {"host", "hbm"}


@dataclass(frozen=True)
class ProjectionPipelineConfig:
    """Policy of the hidden -> QKV -> attention -> output projection pipeline
    (reference src/seqattn_core/config.py:122-142).

    Exact self-attention needs every K/V row before any query can finish, so
    the QKV projection runs as a chunked producer phase, then attention with
    the output projection fused onto each finalized tile.  Additive option:
    ``qkv_residency="hbm"`` keeps the projected Q/K/V in device memory
    instead of staging them in pinned host buffers; attention then reads
    them in place (no Q/K/V PCIe traffic at all) and only the projected
    output crosses the link.
    """

    projection_chunk_tokens: int = 2048
    num_projection_buffers: int = 2
    require_pinned_hidden: bool = True
    pin_qkv: bool = True
    pin_output: bool = True
    enable_nvtx: bool = False
    qkv_residency: str = "host"

    def validate(self) -> None:
        if self.projection_chunk_tokens <= 0:
            raise ValueError("projection_chunk_tokens must be positive")
        if self.num_projection_buffers not in {1, 2, 3}:
            raise ValueError("num_projection_buffers must be 1, 2, or 3")
        if self.qkv_residency not in QKV_RESIDENCIES:
            raise ValueError("qkv_residency must be 'host' or 'hbm'")


__all__ = [
    "BACKENDS",
    "OUTPUT_MODES",
    "PagedAttentionConfig",
    "ProjectionPipelineConfig",
    "QKV_RESIDENCIES",
    "SCHEDULES",
    "StreamingAttentionConfig",
]
