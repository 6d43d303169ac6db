"""Workspace planner: sizes the resident Q super-block and the K/V chunk.

Restates the reference planner (src/seqattn_core/planner.py:11-325) so that a
plan built here for the same shape and budget has the same q_chunk_tokens,
kv_chunk_tokens and estimated bytes (pinned against the reference README's
524,288-token workspace sweep and its planner tests).

* ``estimate_workspace_bytes`` (reference L78-104): resident Q + FP32 state
  (acc + m + l = head_dim + 2 floats per query head) + raw output slots (host
  mode only) + the K/V ring + a fixed 32 MiB margin.
* ``_largest_q_chunk_that_fits`` (L107-155): binary search over block_m
  multiples.
* ``_candidate_cost`` (L158-184): PCIe / state-traffic / launch cost model
  used to pick the K/V chunk jointly with Q.

Measured rates (an addition): ``build_plan(..., rates=PlannerRates(...))``
scores the same candidates with a model of this pipeline built from rates
measured on the device (``measure_planner_rates``): per pass, the K/V copies
of the pass overlap its update launches, so a pass costs the larger of its
H2D time and its kernel time (FLOP at the measured update rate, FP32 state
traffic at the HBM rate, a per-launch overhead), and the plan records the
modeled seconds and the share of the link the plan would use.  Without
rates the reference's fixed constants decide, so the plans (and the golden
rows they are pinned to) are unchanged.

gfx950 specifics: on a ROCm device the launch preset is (128, 64, 4, 2) for
every head_dim: Q chunks align to 128 rows and K/V chunks to the kernel's
64-key LDS tile (a workgroup covers 384 queries for head_dim 72-128 and 256
for head_dim <= 64, and the last workgroup of a chunk is masked, so 128-row
alignment costs at most one partly masked workgroup per chunk).  ``output_mode="host_aliased"`` charges no raw
output slots because the output is finalized into the Q buffer.

Head-group schedule (``config.schedule == "head_groups"``, an addition): the
workspace holds one or two buffer sets, each with every query and key token
of a group of K/V heads (Q, then the output over it; K; V; and V transposed
for head_dim 128).  The planner picks two sets when one K/V head fits twice
(copies of the next unit overlap the current unit's launches), then the
largest group of K/V heads the budget allows, evened out over the units.  The
plan's K/V chunk is the one the default schedule picks for the same budget:
the row sums merge there, so both schedules give the same bits.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch

from .config import StreamingAttentionConfig

FIXED_MARGIN_BYTES = 32 * 2**20
KV_CHUNK_CANDIDATES = (4096, 8192, 16384)

_PORTABLE_KERNEL = (64, 64, 4, 2)
_GFX950_KERNEL = (128, 64, 4, 2)


def _align_down(value: int, alignment: int) -> int:
    return value - value % alignment


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def _charges_output_slots(output_mode: str) -> bool:
    return output_mode == "host"


def _is_rocm_gpu(device: torch.device) -> bool:
    return device.type == "cuda" and torch.version.hip is not None and torch.cuda.is_available()


def _resolve_kernel_config(
    config: StreamingAttentionConfig,
    *,
    device: torch.device,
    head_dim: int,
    dtype: torch.dtype,
) -> StreamingAttentionConfig:
    """Fill unset launch parameters (reference planner.py:19-49).

    Any explicit launch parameter selects the portable baseline for the rest;
    with none set, a ROCm device with float16/bfloat16 inputs gets the gfx950
    preset and everything else the portable one.
    """
    values = (config.block_m, config.block_n, config.num_warps, config.num_stages)
    base = _PORTABLE_KERNEL
    if all(value is None for value in values):
        if _is_rocm_gpu(device) and dtype in {torch.float16, torch.bfloat16}:
            base = _GFX950_KERNEL
    block_m, block_n, num_warps, num_stages = (
        default if value is None else value for value, default in zip(values, base)
    )
    return replace(
        config, block_m=block_m, block_n=block_n, num_warps=num_warps, num_stages=num_stages
    )


@dataclass(frozen=True)
class PlannerRates:
    """Device rates the planner can decide with (bytes and FLOP per second)."""

    h2d_bytes_per_second: float
    update_flops_per_second: float
    hbm_bytes_per_second: float = 5.0e12
    launch_seconds: float = 8e-6


@dataclass(frozen=True)
class AttentionPlan:
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: torch.device
    max_q_tokens: int
    max_kv_tokens: int
    q_chunk_tokens: int
    kv_chunk_tokens: int
    num_kv_buffers: int
    num_output_buffers: int
    output_mode: str
    block_m: int
    block_n: int
    num_warps: int
    num_stages: int
    estimated_workspace_bytes: int
    workspace_budget_bytes: int | None
    # With measured rates only: modeled seconds of one run over max_q_tokens x
    # max_kv_tokens, and the share of the measured H2D rate it keeps busy.
    estimated_seconds: float | None = None
    h2d_link_fraction: float | None = None
    # "q_blocks" or "head_groups"; for head groups, the K/V heads per unit,
    # the buffer sets and each set's transposed-V bytes (0: V read in place).
    schedule: str = "q_blocks"
    head_group_kv_heads: int = 0
    head_group_sets: int = 0
    head_group_vt_bytes: int = 0

    @property
    def group_size(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def q_passes(self) -> int:
        """Passes over K/V for one segment of max_q_tokens queries (one for
        head groups: each unit reads its heads' K/V once)."""
        return math.ceil(self.max_q_tokens / self.q_chunk_tokens)

    @property
    def head_group_units(self) -> int:
        """Units of the head-group schedule (0 for the Q-block schedule)."""
        return len(head_group_unit_sizes(self.kv_heads, self.head_group_kv_heads, self.head_group_sets))


def head_group_unit_sizes(kv_heads: int, group_kv: int, sets: int) -> list[int]:
    """K/V heads of each unit of a head-group run, in order.  With two buffer
    sets the sizes ramp up 1, 2, 4, ... below ``group_kv`` and back down
    ..., 4, 2, 1 at the end, with units of at most ``group_kv`` heads,
    evened out, between: the first unit's copies and the last units' output
    copies are the only ones no launch hides.  Too few heads for both ramps:
    the ramp up, then ``group_kv``.  With one set, units of at most
    ``group_kv``, evened out.  The pipeline (sa_pipeline.cpp,
    head_group_unit_sizes) splits the heads the same way."""
    if group_kv <= 0 or kv_heads <= 0:
        return []
    ramp = []
    if sets > 1:
        size = 1
        while size < group_kv:
            ramp.append(size)
            size *= 2
    if 2 * sum(ramp) > kv_heads:
        sizes, done, size = [], 0, 1 if sets > 1 else group_kv
        while done < kv_heads:
            sizes.append(min(size, group_kv, kv_heads - done))
            done += sizes[-1]
            size = min(2 * size, group_kv)
        return sizes
    middle = kv_heads - 2 * sum(ramp)
    count = -(-middle // group_kv)
    even = [middle // count + (1 if i < middle % count else 0) for i in range(count)] if count else []
    return ramp + even + ramp[::-1]


def estimate_workspace_bytes(
    *,
    q_tokens: int,
    kv_tokens: int,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    num_kv_buffers: int,
    num_output_buffers: int,
    output_mode: str = "host",
) -> int:
    element = _element_size(dtype)
    resident_q = q_tokens * q_heads * head_dim * element
    state = q_tokens * q_heads * (head_dim + 2) * 4  # fp32 acc, m, l
    outputs = (
        num_output_buffers * q_tokens * q_heads * head_dim * element
        if _charges_output_slots(output_mode)
        else 0
    )
    ring = num_kv_buffers * 2 * kv_tokens * kv_heads * head_dim * element
    return resident_q + state + outputs + ring + FIXED_MARGIN_BYTES


def _workspace_for(q_tokens: int, kv_tokens: int, shape: dict, config: StreamingAttentionConfig) -> int:
    return estimate_workspace_bytes(
        q_tokens=q_tokens,
        kv_tokens=kv_tokens,
        num_kv_buffers=config.num_kv_buffers,
        num_output_buffers=config.num_output_buffers,
        output_mode=config.output_mode,
        **shape,
    )


def _largest_q_chunk_that_fits(
    *,
    max_q_tokens: int,
    kv_tokens: int,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    config: StreamingAttentionConfig,
) -> int | None:
    """Largest block_m-aligned resident Q (at least one block) within the budget."""
    shape = {"q_heads": q_heads, "kv_heads": kv_heads, "head_dim": head_dim, "dtype": dtype}
    step = config.block_m
    floor_q = min(step, max_q_tokens)
    budget = config.workspace_budget_bytes
    if budget is None:
        return max_q_tokens
    if _workspace_for(floor_q, kv_tokens, shape, config) > budget:
        return None
    lo, hi, best = floor_q, max_q_tokens, floor_q
    while lo <= hi:
        probe = max(_align_down((lo + hi) // 2, step), floor_q)
        if _workspace_for(probe, kv_tokens, shape, config) <= budget:
            best = probe
            lo = probe + step
        else:
            hi = probe - step
    return min(best, max_q_tokens)


def _candidate_cost(
    *,
    q_chunk: int,
    kv_chunk: int,
    max_q_tokens: int,
    max_kv_tokens: int,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
) -> float:
    """Seconds estimate: K/V re-streaming over PCIe, FP32 state traffic, launches."""
    element = _element_size(dtype)
    passes = math.ceil(max_q_tokens / q_chunk)
    chunks = math.ceil(max_kv_tokens / kv_chunk)
    kv_stream_bytes = passes * 2 * max_kv_tokens * kv_heads * head_dim * element
    state_bytes = chunks * 2 * max_q_tokens * q_heads * (head_dim + 2) * 4
    launches = passes * (chunks + 1)
    # Chunks smaller than 8K pay launch/overlap overhead, larger ones lose
    # ring overlap; both are penalized relative to 8K.
    octaves = math.log2(kv_chunk / 8192)
    overlap = 1.0 + 0.08 * max(-octaves, 0.0) + 0.65 * max(octaves, 0.0)
    return kv_stream_bytes * overlap / 24e9 + state_bytes / 1.2e12 + launches * 8e-6


def modeled_run(
    *,
    q_chunk: int,
    kv_chunk: int,
    max_q_tokens: int,
    max_kv_tokens: int,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    rates: PlannerRates,
) -> tuple[float, float]:
    """(seconds, H2D link fraction) of one non-causal run of the pipeline.

    Each pass copies its Q block once and streams every K/V chunk; a chunk's
    copy overlaps the launches of the previous chunk, so a pass takes the
    larger of its copy time and its kernel time, plus the first chunk's copy,
    which nothing hides when the pass starts.
    """
    element = _element_size(dtype)
    passes = math.ceil(max_q_tokens / q_chunk)
    rows = math.ceil(max_q_tokens / passes)
    chunks = math.ceil(max_kv_tokens / kv_chunk)
    kv_bytes = 2 * max_kv_tokens * kv_heads * head_dim * element
    q_bytes = rows * q_heads * head_dim * element
    h2d_pass = (kv_bytes + q_bytes) / rates.h2d_bytes_per_second
    flop_pass = 4.0 * q_heads * head_dim * rows * max_kv_tokens
    state_pass = chunks * 2 * rows * q_heads * (head_dim + 2) * 4
    kernel_pass = (flop_pass / rates.update_flops_per_second + state_pass / rates.hbm_bytes_per_second
                   + 2 * chunks * rates.launch_seconds)
    first_copy = 2 * min(kv_chunk, max_kv_tokens) * kv_heads * head_dim * element / rates.h2d_bytes_per_second
    seconds = passes * (max(h2d_pass, kernel_pass) + first_copy)
    return seconds, passes * h2d_pass / seconds


def head_group_set_bytes(*, group_kv_heads: int, max_q_tokens: int, max_kv_tokens: int, q_heads: int,
                         kv_heads: int, head_dim: int, dtype: torch.dtype, transposed_v: bool) -> int:
    """Bytes of one head-group buffer set: Q/output, K, V and optionally V
    transposed ([heads][128][keys rounded up to 64], head_dim 128 only)."""
    element = _element_size(dtype)
    group = q_heads // kv_heads
    per_head = max_q_tokens * group * head_dim * element + 2 * max_kv_tokens * head_dim * element
    if transposed_v:
        per_head += 128 * ((max_kv_tokens + 63) // 64 * 64) * 2
    return group_kv_heads * per_head


def _head_group_layout(*, budget: int | None, max_q_tokens: int, max_kv_tokens: int, q_heads: int, kv_heads: int,
                       head_dim: int, dtype: torch.dtype) -> tuple[int, int, bool] | None:
    """(sets, K/V heads per unit, transposed V) for the budget, or None."""
    options = (True, False) if head_dim == 128 else (False,)
    for sets in (2, 1):
        for transposed_v in options:
            per_head = head_group_set_bytes(group_kv_heads=1, max_q_tokens=max_q_tokens, max_kv_tokens=max_kv_tokens,
                                            q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, dtype=dtype,
                                            transposed_v=transposed_v)
            if budget is None:
                fit = kv_heads
            else:
                fit = min(kv_heads, max(budget - FIXED_MARGIN_BYTES, 0) // (sets * per_head))
            if fit >= 1:
                units = math.ceil(kv_heads / fit)
                return sets, math.ceil(kv_heads / units), transposed_v
    return None


def modeled_head_groups(*, max_q_tokens: int, max_kv_tokens: int, q_heads: int, kv_heads: int, head_dim: int,
                        dtype: torch.dtype, group_kv_heads: int, sets: int, rates: PlannerRates) -> tuple[float, float]:
    """(seconds, H2D link fraction) of one non-causal head-group run: every
    unit's launches at the measured rate; with two sets only the first unit's
    copies and the last unit's output copy are exposed, with one set every
    unit's copies are."""
    element = _element_size(dtype)
    sizes = head_group_unit_sizes(kv_heads, group_kv_heads, sets)
    h2d = (max_q_tokens * q_heads + 2 * max_kv_tokens * kv_heads) * head_dim * element
    d2h = max_q_tokens * q_heads * head_dim * element
    kernel = 4.0 * q_heads * head_dim * max_q_tokens * max_kv_tokens / rates.update_flops_per_second
    copy_in = h2d / rates.h2d_bytes_per_second
    copy_out = d2h / rates.h2d_bytes_per_second
    if sets > 1:
        exposed = (copy_in * sizes[0] + copy_out * sizes[-1]) / kv_heads
    else:
        exposed = copy_in + copy_out
    seconds = kernel + exposed + len(sizes) * rates.launch_seconds
    return seconds, copy_in / seconds


def measure_planner_rates(device: torch.device | str = "cuda", *, dtype: torch.dtype = torch.bfloat16,
                          copy_bytes: int = 512 * 2**20) -> PlannerRates:
    """Measure the pinned H2D copy rate and the update kernel's rate on
    ``device`` (a few hundred milliseconds of GPU work)."""
    import time

    from .kernels import update_attention_state

    device = torch.device(device)
    src = torch.empty(copy_bytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(copy_bytes, dtype=torch.uint8, device=device)
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize(device)
    started = time.perf_counter()
    for _ in range(3):
        dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize(device)
    h2d = 3 * copy_bytes / (time.perf_counter() - started)
    del src, dst
    q_rows, keys, heads, dim = 8192, 4096, 32, 128
    q = torch.randn((q_rows, heads, dim), device=device).to(dtype)
    k = torch.randn((keys, heads, dim), device=device).to(dtype)
    v = torch.randn_like(k)
    m = torch.empty((q_rows, heads), device=device)
    l = torch.empty_like(m)
    acc = torch.empty((q_rows, heads, dim), device=device)

    def launch(initialize):
        update_attention_state(q, k, v, m, l, acc, q_tokens=q_rows, kv_tokens=keys, q_local_offset=0,
                               kv_local_offset=0, causal_shift=0, softmax_scale=dim**-0.5, causal=False,
                               initialize=initialize)

    launch(True)
    torch.cuda.synchronize(device)
    started = time.perf_counter()
    for _ in range(5):
        launch(False)
    torch.cuda.synchronize(device)
    flops = 5 * 4.0 * heads * dim * q_rows * keys / (time.perf_counter() - started)
    return PlannerRates(h2d_bytes_per_second=h2d, update_flops_per_second=flops)


def build_plan(
    *,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    device: torch.device | str,
    max_q_tokens: int,
    max_kv_tokens: int,
    config: StreamingAttentionConfig | None = None,
    rates: PlannerRates | None = None,
) -> AttentionPlan:
    """Choose (q_chunk_tokens, kv_chunk_tokens) for a shape and budget.

    ``rates`` (optional): measured device rates; the candidates are then
    ranked by the modeled run time of this pipeline instead of the
    reference's fixed-constant cost.  With ``config.schedule ==
    "head_groups"`` the plan sizes head-group buffer sets instead (module
    docstring); with ``"auto"`` it does so when they fit the budget, the
    output is not a device consumer's and the inputs must be page-locked
    (``require_pinned``).  ``plan.schedule`` names the schedule
    planned."""
    config = StreamingAttentionConfig() if config is None else config
    config.validate()
    device = torch.device(device)
    if device.type == "cuda" and device.index is None and torch.cuda.is_available():
        device = torch.device("cuda", torch.cuda.current_device())
    if q_heads <= 0 or kv_heads <= 0 or q_heads % kv_heads:
        raise ValueError("q_heads must be a positive multiple of kv_heads")
    if head_dim <= 0 or head_dim > 256 or head_dim % 8:
        raise ValueError("head_dim must be a multiple of 8 and at most 256")
    if dtype not in {torch.float16, torch.bfloat16, torch.float32}:
        raise ValueError("dtype must be float16, bfloat16, or float32")
    if max_q_tokens <= 0 or max_kv_tokens <= 0:
        raise ValueError("max_q_tokens and max_kv_tokens must be positive")
    config = _resolve_kernel_config(config, device=device, head_dim=head_dim, dtype=dtype)
    shape = {"q_heads": q_heads, "kv_heads": kv_heads, "head_dim": head_dim, "dtype": dtype}

    if config.kv_chunk_tokens is None:
        kv_options = sorted(
            {max(config.block_n, min(max_kv_tokens, c)) for c in KV_CHUNK_CANDIDATES}
        )
    else:
        kv_options = [min(config.kv_chunk_tokens, max_kv_tokens)]

    scored: list[tuple[float, int, int]] = []
    for kv_option in kv_options:
        kv_chunk = min(max(config.block_n, _align_down(kv_option, config.block_n)), max_kv_tokens)
        if config.q_chunk_tokens is None:
            q_chunk = _largest_q_chunk_that_fits(
                max_q_tokens=max_q_tokens, kv_tokens=kv_chunk, config=config, **shape
            )
            if q_chunk is None:
                continue
        else:
            q_chunk = max(
                min(config.block_m, max_q_tokens),
                _align_down(min(config.q_chunk_tokens, max_q_tokens), config.block_m),
            )
        sizes = {"q_chunk": q_chunk, "kv_chunk": kv_chunk, "max_q_tokens": max_q_tokens,
                 "max_kv_tokens": max_kv_tokens}
        if rates is None:
            cost = _candidate_cost(**sizes, **shape)
        else:
            cost = modeled_run(**sizes, rates=rates, **shape)[0]
        scored.append((cost, q_chunk, kv_chunk))

    # "auto" takes head groups only where the runner can run them: a host
    # output and page-locked inputs (the head columns move by strided copies).
    head_groups = config.schedule == "head_groups" or (
        config.schedule == "auto" and config.output_mode != "device_consumer" and config.require_pinned
        and _head_group_layout(budget=config.workspace_budget_bytes, max_q_tokens=max_q_tokens,
                               max_kv_tokens=max_kv_tokens, **shape) is not None)
    if head_groups:
        # The default schedule's K/V chunk for the same inputs (row sums merge
        # there), rounded to whole 64-key tiles when a segment can be longer.
        if scored:
            kv_chunk = min(scored)[2]
        else:
            kv_chunk = min(max(config.block_n, _align_down(min(kv_options), config.block_n)), max_kv_tokens)
        if kv_chunk % 64 and kv_chunk < max_kv_tokens:
            kv_chunk = max(64, _align_down(kv_chunk, 64))
        return _build_head_group_plan(kv_chunk, config, device, max_q_tokens, max_kv_tokens, shape, rates)
    if not scored:
        smallest = _workspace_for(min(config.block_m, max_q_tokens), min(kv_options), shape, config)
        raise ValueError(
            "workspace budget is too small for one query block and the requested KV buffers: "
            f"need at least {smallest / 2**20:.1f} MiB"
        )
    _, q_chunk, kv_chunk = min(scored)

    estimated = _workspace_for(q_chunk, kv_chunk, shape, config)
    budget = config.workspace_budget_bytes
    if budget is not None and estimated > budget:
        raise ValueError(
            f"requested chunks need {estimated / 2**20:.1f} MiB, exceeding the "
            f"{budget / 2**20:.1f} MiB workspace budget"
        )
    modeled = (None, None)
    if rates is not None:
        modeled = modeled_run(q_chunk=q_chunk, kv_chunk=kv_chunk, max_q_tokens=max_q_tokens,
                              max_kv_tokens=max_kv_tokens, rates=rates, **shape)
    plan = AttentionPlan(
        q_heads=q_heads,
        kv_heads=kv_heads,
        head_dim=head_dim,
        dtype=dtype,
        device=device,
        max_q_tokens=max_q_tokens,
        max_kv_tokens=max_kv_tokens,
        q_chunk_tokens=q_chunk,
        kv_chunk_tokens=kv_chunk,
        num_kv_buffers=config.num_kv_buffers,
        num_output_buffers=config.num_output_buffers,
        output_mode=config.output_mode,
        block_m=config.block_m,
        block_n=config.block_n,
        num_warps=config.num_warps,
        num_stages=config.num_stages,
        estimated_workspace_bytes=estimated,
        workspace_budget_bytes=budget,
        estimated_seconds=modeled[0],
        h2d_link_fraction=modeled[1],
    )
    return plan


def _build_head_group_plan(kv_chunk: int, config: StreamingAttentionConfig, device: torch.device,
                           max_q_tokens: int, max_kv_tokens: int, shape: dict,
                           rates: PlannerRates | None) -> AttentionPlan:
    """The head-group plan for a shape and budget, merging row sums every
    ``kv_chunk`` keys."""
    budget = config.workspace_budget_bytes
    layout = _head_group_layout(budget=budget, max_q_tokens=max_q_tokens, max_kv_tokens=max_kv_tokens, **shape)
    if layout is None:
        need = 1 * head_group_set_bytes(group_kv_heads=1, max_q_tokens=max_q_tokens, max_kv_tokens=max_kv_tokens,
                                        transposed_v=False, **shape) + FIXED_MARGIN_BYTES
        raise ValueError(
            "workspace budget is too small for the head-group schedule (every token of one K/V head): "
            f"need at least {need / 2**20:.1f} MiB"
        )
    sets, group_kv, transposed_v = layout
    set_bytes = head_group_set_bytes(group_kv_heads=group_kv, max_q_tokens=max_q_tokens,
                                     max_kv_tokens=max_kv_tokens, transposed_v=transposed_v, **shape)
    vt_bytes = group_kv * 128 * ((max_kv_tokens + 63) // 64 * 64) * 2 if transposed_v else 0
    modeled = (None, None)
    if rates is not None:
        modeled = modeled_head_groups(max_q_tokens=max_q_tokens, max_kv_tokens=max_kv_tokens, group_kv_heads=group_kv,
                                      sets=sets, rates=rates, **shape)
    return AttentionPlan(
        q_heads=shape["q_heads"],
        kv_heads=shape["kv_heads"],
        head_dim=shape["head_dim"],
        dtype=shape["dtype"],
        device=device,
        max_q_tokens=max_q_tokens,
        max_kv_tokens=max_kv_tokens,
        q_chunk_tokens=max_q_tokens,
        kv_chunk_tokens=kv_chunk,
        num_kv_buffers=config.num_kv_buffers,
        num_output_buffers=config.num_output_buffers,
        output_mode=config.output_mode,
        block_m=config.block_m,
        block_n=config.block_n,
        num_warps=config.num_warps,
        num_stages=config.num_stages,
        estimated_workspace_bytes=sets * set_bytes + FIXED_MARGIN_BYTES,
        workspace_budget_bytes=budget,
        estimated_seconds=modeled[0],
        h2d_link_fraction=modeled[1],
        schedule="head_groups",
        head_group_kv_heads=group_kv,
        head_group_sets=sets,
        head_group_vt_bytes=vt_bytes,
    )


__all__ = [
    "AttentionPlan",
    "PlannerRates",
    "build_plan",
    "estimate_workspace_bytes",
    "head_group_set_bytes",
    "measure_planner_rates",
    "head_group_unit_sizes",
    "modeled_head_groups",
    "modeled_run",
]
