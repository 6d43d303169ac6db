"""GPU parity of the head-group schedule (``schedule="head_groups"``).

A head-group run keeps every token of a group of K/V heads (and their query
heads) in HBM, copies each byte of Q, K and V once, and makes one fused update
launch per (unit, segment).  Its output and LSE must equal the default
Q-block schedule's bit for bit for the same K/V chunk (the row sums merge at
the same boundaries), and match the FP32 oracle within the tolerances of
tests/test_gpu_streaming.py.  Layouts are forced through the plan (K/V heads
per unit, one or two buffer sets, transposed V or V read in place) so that
every path of the schedule runs: units that alternate streams, a short last
unit, a single unit holding every head, empty and ragged segments, GQA,
causal masks with rows that see no key, fp16, and the 32-query kernel.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from seqattn import StreamingAttentionConfig, StreamingAttentionRunner, StreamingAttentionStats, build_plan
from seqattn.planner import head_group_unit_sizes
from test_gpu_streaming import announce, check, oracle, pinned_randn

pytestmark = pytest.mark.gpu


def run_plan(plan, config, q, k, v, cu_q, cu_k, causal):
    runner = StreamingAttentionRunner(plan, config)
    stats = StreamingAttentionStats()
    try:
        out, lse = runner(q, k, v, cu_q, cu_k, causal=causal, return_lse=True, stats=stats)
    finally:
        runner.close()
    return out, lse, stats


def head_group_plan(q, k, config, *, group_kv, sets, transposed_v):
    plan = build_plan(q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=q.shape[2], dtype=q.dtype, device="cuda",
                      max_q_tokens=q.shape[0], max_kv_tokens=k.shape[0],
                      config=dataclasses.replace(config, schedule="head_groups"))
    vt_bytes = group_kv * 128 * (-(-k.shape[0] // 64) * 64) * 2 if transposed_v else 0
    return dataclasses.replace(plan, head_group_kv_heads=group_kv, head_group_sets=sets,
                               head_group_vt_bytes=vt_bytes)


CASES = [
    # (dtype, head_dim, q_heads, kv_heads, K/V heads per unit, sets, transposed V)
    (torch.bfloat16, 128, 4, 4, 1, 2, True),    # one head per unit, units alternate streams
    (torch.bfloat16, 128, 4, 4, 3, 1, False),   # one set, a short last unit
    (torch.bfloat16, 128, 4, 4, 4, 2, True),    # a single unit holds every head
    (torch.bfloat16, 128, 8, 2, 1, 2, False),   # GQA, V read in place
    (torch.float16, 128, 6, 3, 2, 2, True),     # fp16, GQA, short last unit
    (torch.bfloat16, 96, 4, 2, 1, 2, False),    # a partial d block of the 48-query kernel
    (torch.bfloat16, 64, 6, 3, 2, 1, False),    # the 32-query kernel
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{str(c[0])[6:]}-d{c[1]}-h{c[2]}/{c[3]}-g{c[4]}-s{c[5]}-vt{int(c[6])}")
def test_head_groups_bit_identical_to_q_blocks(case, causal):
    dtype, head_dim, q_heads, kv_heads, group_kv, sets, transposed_v = case
    announce(f"head groups {case} causal={causal}")
    gen = torch.Generator().manual_seed(50 + head_dim + q_heads)
    # Ragged segments: an empty one, one with fewer keys than queries (under
    # the causal rule its first rows see no key), one longer than several
    # chunks with a partial last chunk.
    cu_q = torch.tensor([0, 700, 700, 1300, 2500], dtype=torch.int32)
    cu_k = torch.tensor([0, 900, 950, 1450, 2550], dtype=torch.int32)
    q = pinned_randn((2500, q_heads, head_dim), dtype, gen)
    k = pinned_randn((2550, kv_heads, head_dim), dtype, gen)
    v = pinned_randn((2550, kv_heads, head_dim), dtype, gen)
    config = StreamingAttentionConfig(backend="hip", q_chunk_tokens=512, kv_chunk_tokens=256)
    base = build_plan(q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, dtype=dtype, device="cuda",
                      max_q_tokens=2500, max_kv_tokens=2550, config=config)
    out_b, lse_b, st_b = run_plan(base, config, q, k, v, cu_q, cu_k, causal)
    plan = head_group_plan(q, k, config, group_kv=group_kv, sets=sets, transposed_v=transposed_v)
    assert plan.kv_chunk_tokens == base.kv_chunk_tokens == 256
    hg_config = dataclasses.replace(config, schedule="head_groups")
    out_h, lse_h, st_h = run_plan(plan, hg_config, q, k, v, cu_q, cu_k, causal)
    torch.testing.assert_close(out_h, out_b, atol=0, rtol=0)
    torch.testing.assert_close(lse_h, lse_b, atol=0, rtol=0)
    element = q.element_size()
    assert st_h.h2d_bytes == (q.numel() + k.numel() + v.numel()) * element
    assert st_h.d2h_bytes == st_b.d2h_bytes == q.numel() * element
    assert st_h.q_chunks == plan.head_group_units == len(head_group_unit_sizes(kv_heads, group_kv, sets))
    assert st_h.max_resident_q_tokens == 2500
    ref_o, ref_l = oracle(q, k, v, cu_q, cu_k, q_chunk=512, kv_chunk=256, causal=causal)
    check(out_h, lse_h, ref_o, ref_l)


def test_head_groups_repeated_runs_reuse_the_sets():
    """Three runs on one runner: later runs wait for the sets' previous output
    copies and give the same bits; a smaller second input uses a prefix of
    the sets."""
    announce("head groups repeated runs")
    gen = torch.Generator().manual_seed(71)
    q = pinned_randn((1500, 6, 128), torch.bfloat16, gen)
    k = pinned_randn((1400, 6, 128), torch.bfloat16, gen)
    v = pinned_randn((1400, 6, 128), torch.bfloat16, gen)
    # 40 MiB: the fixed 32 MiB margin plus two sets of two K/V heads; the
    # units ramp up from one head: 1, 2, 2, 1.
    config = StreamingAttentionConfig(backend="hip", kv_chunk_tokens=512, schedule="head_groups",
                                      workspace_budget_bytes=40 * 2**20)
    plan = build_plan(q_heads=6, kv_heads=6, head_dim=128, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=1500, max_kv_tokens=1400, config=config)
    assert (plan.schedule, plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_units) == (
        "head_groups", 2, 2, 4)
    runner = StreamingAttentionRunner(plan, config)
    try:
        cu_q = torch.tensor([0, 1500], dtype=torch.int32)
        cu_k = torch.tensor([0, 1400], dtype=torch.int32)
        first = runner(q, k, v, cu_q, cu_k, return_lse=True)
        small = runner(q[:600], k[:500], v[:500], torch.tensor([0, 600], dtype=torch.int32),
                       torch.tensor([0, 500], dtype=torch.int32), causal=True, return_lse=True)
        again = runner(q, k, v, cu_q, cu_k, return_lse=True)
    finally:
        runner.close()
    torch.testing.assert_close(again[0], first[0], atol=0, rtol=0)
    torch.testing.assert_close(again[1], first[1], atol=0, rtol=0)
    ref_o, ref_l = oracle(q, k, v, cu_q, cu_k, q_chunk=1500, kv_chunk=512, causal=False)
    check(first[0], first[1], ref_o, ref_l)
    ref_o, ref_l = oracle(q[:600], k[:500], v[:500], [0, 600], [0, 500], q_chunk=600, kv_chunk=512, causal=True)
    check(small[0], small[1], ref_o, ref_l)


def test_auto_schedule_runs_head_groups_or_q_blocks_with_the_same_bits():
    """schedule="auto": head groups where a unit fits the budget (page-locked
    inputs), Q blocks with pageable inputs allowed; both give the bits of an
    explicit Q-block run at the same K/V chunk."""
    announce("auto schedule")
    gen = torch.Generator().manual_seed(73)
    q = pinned_randn((1500, 6, 128), torch.bfloat16, gen)
    k = pinned_randn((1400, 6, 128), torch.bfloat16, gen)
    v = pinned_randn((1400, 6, 128), torch.bfloat16, gen)
    cu_q = torch.tensor([0, 400, 1500], dtype=torch.int32)
    cu_k = torch.tensor([0, 300, 1400], dtype=torch.int32)
    shape = dict(q_heads=6, kv_heads=6, head_dim=128, dtype=torch.bfloat16, device="cuda", max_q_tokens=1500,
                 max_kv_tokens=1400)
    results = {}
    for name, extra in (("q_blocks", {}), ("auto", {"schedule": "auto"}),
                        ("auto_pageable", {"schedule": "auto", "require_pinned": False})):
        config = StreamingAttentionConfig(backend="hip", kv_chunk_tokens=512, workspace_budget_bytes=40 * 2**20,
                                          **extra)
        plan = build_plan(config=config, **shape)
        expected = "head_groups" if name == "auto" else "q_blocks"
        assert plan.schedule == expected, name
        inputs = (q, k, v) if name != "auto_pageable" else (q.clone(), k.clone(), v.clone())
        out, lse, _ = run_plan(plan, config, *inputs, cu_q, cu_k, True)
        results[name] = (out, lse)
    for name in ("auto", "auto_pageable"):
        torch.testing.assert_close(results[name][0], results["q_blocks"][0], atol=0, rtol=0)
        torch.testing.assert_close(results[name][1], results["q_blocks"][1], atol=0, rtol=0)
    ref_o, ref_l = oracle(q, k, v, cu_q, cu_k, q_chunk=1500, kv_chunk=512, causal=True)
    check(results["auto"][0], results["auto"][1], ref_o, ref_l)


def test_head_groups_device_inputs_device_output_and_consumers():
    """On a head-group runner: device-resident inputs run the fused launch,
    and a device out is written by the unit launches (no output copy), both
    bit-identical to the host run; device consumers are refused before
    anything runs."""
    announce("head groups device inputs")
    gen = torch.Generator().manual_seed(73)
    q = pinned_randn((800, 4, 128), torch.bfloat16, gen)
    k = pinned_randn((900, 2, 128), torch.bfloat16, gen)
    v = pinned_randn((900, 2, 128), torch.bfloat16, gen)
    cu_q = torch.tensor([0, 300, 800], dtype=torch.int32)
    cu_k = torch.tensor([0, 400, 900], dtype=torch.int32)
    config = StreamingAttentionConfig(backend="hip", kv_chunk_tokens=256, schedule="head_groups")
    plan = build_plan(q_heads=4, kv_heads=2, head_dim=128, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=800, max_kv_tokens=900, config=config)
    runner = StreamingAttentionRunner(plan, config)
    try:
        out, lse = runner(q, k, v, cu_q, cu_k, causal=True, return_lse=True)
        out_d, lse_d = runner(q.cuda(), k.cuda(), v.cuda(), cu_q, cu_k, causal=True, return_lse=True)
        dev_out = torch.full(q.shape, float("nan"), dtype=q.dtype, device="cuda")
        stats = StreamingAttentionStats()
        _, lse_o = runner(q, k, v, cu_q, cu_k, causal=True, out=dev_out, return_lse=True, stats=stats)
        torch.cuda.synchronize()
        assert stats.d2h_bytes == 0 and stats.h2d_bytes == (q.numel() + k.numel() + v.numel()) * 2
        torch.testing.assert_close(dev_out.cpu(), out, atol=0, rtol=0)
        torch.testing.assert_close(lse_o.cpu(), lse.cpu(), atol=0, rtol=0)
        with pytest.raises(ValueError, match="q_blocks"):
            runner.run_with_device_output(q, k, v, cu_q, cu_k, output_transform=None,
                                          out=torch.empty(q.shape, dtype=q.dtype, device="cuda"))
    finally:
        runner.close()
    torch.testing.assert_close(out_d.cpu(), out, atol=0, rtol=0)
    torch.testing.assert_close(lse_d.cpu(), lse.cpu(), atol=0, rtol=0)
    ref_o, ref_l = oracle(q, k, v, cu_q, cu_k, q_chunk=800, kv_chunk=256, causal=True)
    check(out, lse, ref_o, ref_l)


@pytest.mark.parametrize("sets", [1, 2])
def test_head_groups_pageable_output_through_staging(sets):
    """A pageable out (pin_output=False) is written through the pipeline's
    page-locked staging in row chunks, bit-identical to a page-locked out;
    GQA, two segments, causal."""
    announce(f"head groups pageable output sets={sets}")
    gen = torch.Generator().manual_seed(79)
    q = pinned_randn((3000, 8, 128), torch.bfloat16, gen)
    k = pinned_randn((2800, 4, 128), torch.bfloat16, gen)
    v = pinned_randn((2800, 4, 128), torch.bfloat16, gen)
    cu_q = torch.tensor([0, 1000, 3000], dtype=torch.int32)
    cu_k = torch.tensor([0, 900, 2800], dtype=torch.int32)
    base = StreamingAttentionConfig(backend="hip", kv_chunk_tokens=512, schedule="head_groups")
    plan = build_plan(q_heads=8, kv_heads=4, head_dim=128, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=3000, max_kv_tokens=2800, config=base)
    plan = dataclasses.replace(plan, head_group_kv_heads=1, head_group_sets=sets,
                               head_group_vt_bytes=128 * 2816 * 2)
    results = []
    for pinned in (True, False):
        config = dataclasses.replace(base, pin_output=pinned)
        runner = StreamingAttentionRunner(plan, config)
        out = torch.empty(q.shape, dtype=q.dtype, pin_memory=pinned)
        try:
            lse = runner(q, k, v, cu_q, cu_k, causal=True, out=out, return_lse=True)[1]
        finally:
            runner.close()
        assert out.is_pinned() == pinned
        results.append((out, lse))
    torch.testing.assert_close(results[1][0], results[0][0], atol=0, rtol=0)
    torch.testing.assert_close(results[1][1], results[0][1], atol=0, rtol=0)
    ref_o, ref_l = oracle(q, k, v, cu_q, cu_k, q_chunk=3000, kv_chunk=512, causal=True)
    check(results[1][0], results[1][1], ref_o, ref_l)
