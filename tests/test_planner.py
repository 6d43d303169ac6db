"""Planner parity: reference known answers (tests/test_planner.py of the
reference) and the published resident-Q rows (README.md:61-68, perf doc)."""

import json
import math
from pathlib import Path

import pytest
import torch

from seqattn import StreamingAttentionConfig, build_plan
from seqattn.planner import estimate_workspace_bytes, head_group_unit_sizes

GOLDEN = json.loads((Path(__file__).parent / "golden" / "planner_reference_rows.json").read_text())


def test_planner_uses_largest_query_chunk_that_fits_budget():
    shape = {"q_heads": 16, "kv_heads": 4, "head_dim": 64, "dtype": torch.bfloat16,
             "num_kv_buffers": 2, "num_output_buffers": 2}
    budget = estimate_workspace_bytes(q_tokens=512, kv_tokens=256, **shape)
    plan = build_plan(
        q_heads=16, kv_heads=4, head_dim=64, dtype=torch.bfloat16, device="cpu",
        max_q_tokens=2048, max_kv_tokens=2048,
        config=StreamingAttentionConfig(workspace_budget_bytes=budget, kv_chunk_tokens=256,
                                        num_output_buffers=2),
    )
    assert plan.q_chunk_tokens == 512
    assert plan.estimated_workspace_bytes <= budget
    assert plan.group_size == 4


def test_planner_rejects_invalid_gqa_ratio():
    with pytest.raises(ValueError, match="multiple"):
        build_plan(q_heads=6, kv_heads=4, head_dim=64, dtype=torch.bfloat16, device="cpu",
                   max_q_tokens=16, max_kv_tokens=16)


def test_planner_rejects_explicit_chunks_over_budget():
    with pytest.raises(ValueError, match="exceeding"):
        build_plan(q_heads=16, kv_heads=4, head_dim=64, dtype=torch.bfloat16, device="cpu",
                   max_q_tokens=2048, max_kv_tokens=2048,
                   config=StreamingAttentionConfig(workspace_budget_bytes=40 * 2**20,
                                                   q_chunk_tokens=2048, kv_chunk_tokens=1024))


def test_planner_rejects_budget_below_one_block():
    with pytest.raises(ValueError, match="too small"):
        build_plan(q_heads=56, kv_heads=56, head_dim=128, dtype=torch.bfloat16, device="cpu",
                   max_q_tokens=65536, max_kv_tokens=65536,
                   config=StreamingAttentionConfig(workspace_budget_bytes=40 * 2**20))


def test_joint_planner_prefers_8k_kv_and_large_resident_q_for_h3_shape():
    plan = build_plan(q_heads=56, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cpu",
                      max_q_tokens=61_312, max_kv_tokens=61_312,
                      config=StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30,
                                                      output_mode="device_consumer"))
    assert plan.kv_chunk_tokens == 8192
    assert 43_000 <= plan.q_chunk_tokens <= 50_000
    assert plan.estimated_workspace_bytes <= 2 * 2**30


def test_device_consumer_plan_does_not_charge_raw_output_buffer():
    shape = {"q_tokens": 512, "kv_tokens": 256, "q_heads": 16, "kv_heads": 4, "head_dim": 64,
             "dtype": torch.bfloat16, "num_kv_buffers": 2, "num_output_buffers": 2}
    host = estimate_workspace_bytes(**shape, output_mode="host")
    consumer = estimate_workspace_bytes(**shape, output_mode="device_consumer")
    aliased = estimate_workspace_bytes(**shape, output_mode="host_aliased")
    assert host - consumer == 2 * 512 * 16 * 64 * 2
    assert aliased == consumer


def test_default_kernel_profile_is_portable_on_cpu():
    plan = build_plan(q_heads=8, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cpu",
                      max_q_tokens=1024, max_kv_tokens=1024)
    assert (plan.block_m, plan.block_n, plan.num_warps, plan.num_stages) == (64, 64, 4, 2)


def test_explicit_kernel_parameter_uses_portable_defaults_for_the_rest():
    plan = build_plan(q_heads=8, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cpu",
                      max_q_tokens=1024, max_kv_tokens=1024,
                      config=StreamingAttentionConfig(block_m=32))
    assert (plan.block_m, plan.block_n, plan.num_warps, plan.num_stages) == (32, 64, 4, 2)


@pytest.mark.parametrize("row", GOLDEN["sweep_524k"]["rows"], ids=lambda r: f"{r['workspace_gib']}GiB")
def test_planner_reproduces_published_524k_sweep(row):
    g = GOLDEN["sweep_524k"]
    plan = build_plan(
        q_heads=g["q_heads"], kv_heads=g["kv_heads"], head_dim=g["head_dim"], dtype=torch.bfloat16,
        device="cpu", max_q_tokens=g["tokens"], max_kv_tokens=g["tokens"],
        config=StreamingAttentionConfig(workspace_budget_bytes=row["workspace_gib"] * 2**30,
                                        block_m=g["block_m"], kv_chunk_tokens=g["kv_chunk_tokens"]),
    )
    assert plan.q_chunk_tokens == row["resident_q"]
    assert plan.q_passes == row["q_passes"]
    qkv_bytes = g["tokens"] * g["q_heads"] * g["head_dim"] * 2
    h2d_gib = (qkv_bytes + plan.q_passes * 2 * qkv_bytes) / 2**30
    assert round(h2d_gib) == row["h2d_gib"]


@pytest.mark.parametrize("row", GOLDEN["kv_chunk_61k"]["rows"], ids=lambda r: str(r["kv_chunk_tokens"]))
def test_planner_reproduces_published_61k_kv_chunk_rows(row):
    g = GOLDEN["kv_chunk_61k"]
    plan = build_plan(
        q_heads=g["q_heads"], kv_heads=g["kv_heads"], head_dim=g["head_dim"], dtype=torch.bfloat16,
        device="cpu", max_q_tokens=g["tokens"], max_kv_tokens=g["tokens"],
        config=StreamingAttentionConfig(workspace_budget_bytes=g["workspace_gib"] * 2**30,
                                        block_m=g["block_m"], kv_chunk_tokens=row["kv_chunk_tokens"]),
    )
    assert plan.q_chunk_tokens == row["resident_q"]


def test_host_aliased_output_grows_resident_q():
    common = dict(q_heads=56, kv_heads=56, head_dim=128, dtype=torch.bfloat16, device="cpu",
                  max_q_tokens=524288, max_kv_tokens=524288)
    host = build_plan(**common, config=StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30, block_m=128))
    aliased = build_plan(**common, config=StreamingAttentionConfig(
        workspace_budget_bytes=2 * 2**30, block_m=128, output_mode="host_aliased"))
    assert aliased.q_chunk_tokens > host.q_chunk_tokens
    assert aliased.q_passes < host.q_passes
    assert aliased.estimated_workspace_bytes <= 2 * 2**30


def test_planned_workspace_is_monotone_in_budget():
    previous = 0
    for gib in (1, 2, 4, 8, 14):
        plan = build_plan(q_heads=56, kv_heads=56, head_dim=128, dtype=torch.bfloat16, device="cpu",
                          max_q_tokens=524288, max_kv_tokens=524288,
                          config=StreamingAttentionConfig(workspace_budget_bytes=gib * 2**30,
                                                          block_m=128, kv_chunk_tokens=8192))
        assert plan.q_chunk_tokens % 128 == 0
        assert plan.q_chunk_tokens >= previous
        assert plan.estimated_workspace_bytes <= gib * 2**30
        # one more block would not fit
        bigger = estimate_workspace_bytes(
            q_tokens=plan.q_chunk_tokens + 128, kv_tokens=8192, q_heads=56, kv_heads=56, head_dim=128,
            dtype=torch.bfloat16, num_kv_buffers=2, num_output_buffers=1)
        assert plan.q_chunk_tokens == 524288 or bigger > gib * 2**30
        previous = plan.q_chunk_tokens
    assert math.ceil(524288 / previous) == 3


def test_measured_rates_pick_fewest_passes_on_a_slow_link_and_large_chunks_when_kernel_bound():
    from seqattn.planner import PlannerRates, modeled_run

    shape = dict(q_heads=56, kv_heads=56, head_dim=128, dtype=torch.bfloat16, device="cpu",
                 max_q_tokens=524_288, max_kv_tokens=524_288)
    config = StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30)
    slow = build_plan(**shape, config=config, rates=PlannerRates(h2d_bytes_per_second=1e9,
                                                                 update_flops_per_second=1.1e15))
    fast = build_plan(**shape, config=config, rates=PlannerRates(h2d_bytes_per_second=1e15,
                                                                 update_flops_per_second=1.1e15))
    # A slow link makes re-streaming K/V dominate: the smallest ring and so the
    # largest Q block (fewest passes) wins.  A kernel-bound run saves FP32
    # state traffic and launches with the largest chunk.
    assert slow.kv_chunk_tokens == 4096 and slow.h2d_link_fraction > 0.99
    assert fast.kv_chunk_tokens == 16384 and fast.h2d_link_fraction < 0.01
    for plan in (slow, fast):
        assert plan.estimated_workspace_bytes <= 2 * 2**30
        seconds, fraction = modeled_run(q_chunk=plan.q_chunk_tokens, kv_chunk=plan.kv_chunk_tokens,
                                        max_q_tokens=524_288, max_kv_tokens=524_288, q_heads=56, kv_heads=56,
                                        head_dim=128, dtype=torch.bfloat16,
                                        rates=PlannerRates(h2d_bytes_per_second=1e9, update_flops_per_second=1.1e15)
                                        if plan is slow else
                                        PlannerRates(h2d_bytes_per_second=1e15, update_flops_per_second=1.1e15))
        assert seconds == plan.estimated_seconds and 0 < fraction <= 1
    # The modeled kernel time of a kernel-bound run is at least its FLOP at the rate.
    assert fast.estimated_seconds >= 4 * 56 * 128 * 524_288**2 / 1.1e15
    # Without rates the reference's choice stands (README.md:62).
    plain = build_plan(**shape, config=config)
    assert (plain.q_chunk_tokens, plain.kv_chunk_tokens, plain.estimated_seconds) == (28_416, 8_192, None)


# Head-group schedule (config.schedule == "head_groups"): buffer sets holding
# every token of a group of K/V heads.  Expected values are worked out from
# the set layout: per K/V head, Q and the output over it (tokens x group x D
# x 2 bytes), K and V (tokens x D x 2 each) and, for head_dim 128, V
# transposed ([128][tokens rounded up to 64] x 2 bytes).


def _hg(budget_gib, *, n=524_288, heads=56, kv_heads=None, head_dim=128, **cfg):
    config = StreamingAttentionConfig(workspace_budget_bytes=int(budget_gib * 2**30), schedule="head_groups", **cfg)
    return build_plan(q_heads=heads, kv_heads=kv_heads or heads, head_dim=head_dim, dtype=torch.bfloat16,
                      device="cpu", max_q_tokens=n, max_kv_tokens=n, config=config)


def test_head_group_plan_at_the_benchmark_shape():
    plan = _hg(2)
    per_head = 524_288 * 128 * 2  # one tensor's bytes for one head
    assert plan.schedule == "head_groups"
    # Two sets of one head with V transposed: 2 x 4 x 134 MB = 1.07 GB; two
    # heads per set would need 2.15 GB.
    assert (plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_units) == (2, 1, 56)
    assert plan.head_group_vt_bytes == per_head
    assert plan.estimated_workspace_bytes == 2 * 4 * per_head + 32 * 2**20 <= 2 * 2**30
    # The default schedule's K/V chunk (row sums merge there): same bits.
    assert plan.kv_chunk_tokens == 8192
    assert plan.q_chunk_tokens == 524_288 and plan.q_passes == 1


def test_head_group_plan_drops_the_transposed_copy_before_the_second_set():
    # 1 GiB: two sets with V transposed (1.07 GB + margin) do not fit, two
    # without it (0.81 GB) do; the K/V chunk follows the default plan (4,096).
    plan = _hg(1)
    assert (plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_vt_bytes) == (2, 1, 0)
    assert plan.kv_chunk_tokens == 4096
    # 0.5 GiB: one set of Q, K and V (403 MB) is all that fits.
    plan = _hg(0.5)
    assert (plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_vt_bytes) == (1, 1, 0)


def test_head_group_units_are_evened_out():
    # 14 GiB fits 12 heads per set pair (12 x 1.07 GB = 12.9 GB); 56 heads in
    # ceil(56 / 12) = 5 units, evened out to ceil(56 / 5) = 12 per unit.  The
    # run ramps the unit sizes up from one head and back down to one (only
    # the first unit's copies and the last units' output copies are
    # exposed), with the 42 heads between in units of at most 12, evened out.
    plan = _hg(14)
    assert (plan.head_group_kv_heads, plan.head_group_units) == (12, 11)
    assert head_group_unit_sizes(56, 12, 2) == [1, 2, 4, 8, 9, 9, 8, 8, 4, 2, 1]
    # Too few heads for both ramps: up only.  One set (no copy overlaps a
    # launch): no ramp.
    assert head_group_unit_sizes(8, 8, 2) == [1, 2, 4, 1]
    assert head_group_unit_sizes(56, 12, 1) == [12, 11, 11, 11, 11]
    assert head_group_unit_sizes(56, 1, 2) == [1] * 56
    # GQA: a unit takes its K/V heads' query heads too (8 query heads per
    # K/V head here), and the transposed copy is per K/V head.
    plan = _hg(2, heads=64, kv_heads=8)
    per_kv_head = 524_288 * 128 * 2 * (8 + 2 + 1)
    fit = (2 * 2**30 - 32 * 2**20) // (2 * per_kv_head)
    assert fit == 0
    # one K/V head with its 8 query heads is 1.48 GB per set: one set only.
    assert (plan.head_group_sets, plan.head_group_kv_heads) == (1, 1)


def test_head_group_plan_without_budget_holds_every_head_and_rejects_tiny_budgets():
    plan = build_plan(q_heads=8, kv_heads=2, head_dim=64, dtype=torch.bfloat16, device="cpu", max_q_tokens=4096,
                      max_kv_tokens=4096, config=StreamingAttentionConfig(schedule="head_groups"))
    assert (plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_units, plan.head_group_vt_bytes) == (
        2, 2, 2, 0)
    with pytest.raises(ValueError, match="too small for the head-group schedule"):
        _hg(0.25)


def test_head_group_chunk_is_rounded_to_whole_tiles_when_segments_can_be_longer():
    config = StreamingAttentionConfig(schedule="head_groups", kv_chunk_tokens=1000, block_n=16)
    plan = build_plan(q_heads=4, kv_heads=4, head_dim=64, dtype=torch.bfloat16, device="cpu", max_q_tokens=5000,
                      max_kv_tokens=5000, config=config)
    assert plan.kv_chunk_tokens == 960
    # A chunk covering every key needs no merge boundary and is kept.
    plan = build_plan(q_heads=4, kv_heads=4, head_dim=64, dtype=torch.bfloat16, device="cpu", max_q_tokens=912,
                      max_kv_tokens=912, config=config)
    assert plan.kv_chunk_tokens == 912


def test_schedule_validation():
    with pytest.raises(ValueError, match="schedule must be"):
        StreamingAttentionConfig(schedule="tiles").validate()
    with pytest.raises(ValueError, match="device_consumer"):
        StreamingAttentionConfig(schedule="head_groups", output_mode="device_consumer").validate()
    StreamingAttentionConfig(schedule="head_groups", output_mode="host_aliased").validate()


def test_auto_schedule_plans_head_groups_when_they_fit():
    config = StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30, schedule="auto")
    shape = dict(q_heads=56, kv_heads=56, head_dim=128, dtype=torch.bfloat16, device="cpu", max_q_tokens=524_288,
                 max_kv_tokens=524_288)
    plan = build_plan(config=config, **shape)
    assert (plan.schedule, plan.head_group_kv_heads, plan.head_group_sets) == ("head_groups", 1, 2)
    # A device consumer finishes Q tiles: Q blocks, the reference's plan.
    consumer = StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30, schedule="auto",
                                        output_mode="device_consumer")
    plan = build_plan(config=consumer, **shape)
    reference = build_plan(config=StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30,
                                                           output_mode="device_consumer"), **shape)
    assert plan.schedule == "q_blocks" and plan == reference
    # 320 MiB holds no head of 524,288 tokens (403 MB without V transposed,
    # plus the margin): Q blocks.
    small = StreamingAttentionConfig(workspace_budget_bytes=320 * 2**20, schedule="auto")
    plan = build_plan(config=small, **shape)
    assert plan.schedule == "q_blocks"
    assert plan.q_chunk_tokens == build_plan(config=StreamingAttentionConfig(workspace_budget_bytes=320 * 2**20),
                                             **shape).q_chunk_tokens
    # Pageable inputs allowed (require_pinned=False): head columns cannot
    # move by strided copies from them, so Q blocks.
    pageable = StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30, schedule="auto", require_pinned=False)
    assert build_plan(config=pageable, **shape).schedule == "q_blocks"


def test_head_group_unit_sizes_cover_every_head_within_the_group_size():
    for kv_heads in range(1, 65):
        for group_kv in range(1, 17):
            for sets in (1, 2):
                sizes = head_group_unit_sizes(kv_heads, group_kv, sets)
                assert sum(sizes) == kv_heads and all(1 <= s <= group_kv for s in sizes)
                if sets == 2:
                    assert sizes[0] == 1
                else:
                    assert len(sizes) == -(-kv_heads // group_kv)
