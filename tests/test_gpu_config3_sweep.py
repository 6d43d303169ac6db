"""GPU parity of the 524,288-token workload at every HBM workspace of its sweep.

524,288 tokens x 56 heads x head_dim 128, bf16, non-causal, Q/K/V ~ N(0,1)
in caller-owned pinned DRAM, output back to pinned DRAM, the LSE of every
row written.  The workspace budget is swept over 1, 2, 4, 8 and 14 GiB (the
reference's dram_workspace_sweep protocol, benchmarks/dram_workspace_sweep.py:
99-171); each budget gives the planner a different decomposition, and the
test asserts the planner's choice for it (from 2 GiB up the reference's
published rows, README.md:61-68) before running one step.  O and the
natural-log LSE are compared with the FP32 oracle on the reference's
large-tier signature rows {0, N/4, N/2, 3N/4, N-1}
(benchmarks/large_tier_comparison.py:62-66) plus 1,024 seeded-random rows,
every head, against every key, with the oracle chunking K/V like the plan.  Tolerances: O max-abs <= 2e-2, LSE max-abs <= 1e-3, O
relative L2 <= 5e-3, every element within 2^-5 (|ref| + rms(ref)).

The inputs (30 GB page-locked with the output) are made once for the module
and released when it ends.

The head-group schedule (``schedule="head_groups"``: every token of one K/V
head resident at once, Q/K/V copied once) runs the same step at 1 and 2 GiB:
its sampled rows must equal the default schedule's at the same budget bit for
bit and match the oracle.
"""

from __future__ import annotations

import pytest
import torch

from seqattn import StreamingAttentionConfig, StreamingAttentionRunner, StreamingAttentionStats, build_plan
from seeded import check_parity, oracle_rows, release_host_memory, seeded_qkv, signature_and_random_rows

pytestmark = pytest.mark.gpu

N, H, D = 524_288, 56, 128

# Workspace (GiB) -> the planner's (q_chunk_tokens, kv_chunk_tokens, q_passes)
# for this shape on a ROCm device, where the launch preset has block_m 128
# like the reference's published rows.  From 2 GiB up the Q blocks equal
# README.md:61-68 (28,416 / 65,536 / 139,904 / 251,392 at K/V chunk 8,192);
# at 1 GiB the automatic K/V chunk is 4,096 (README's row fixes 8,192).
SWEEP = {
    1: (13_824, 4_096, 38),
    2: (28_416, 8_192, 19),
    4: (65_536, 8_192, 8),
    8: (139_904, 8_192, 4),
    14: (251_392, 8_192, 3),
}


# Sampled output rows and LSE of the default schedule per budget, for the
# head-group runs' bit-identity check.
SNAPSHOTS: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}


@pytest.fixture(scope="module")
def sweep_inputs():
    print(f"[gpu case] config 3 sweep inputs: {N} x {H} x {D} bf16 pinned, oracle rows", flush=True)
    q, k, v = seeded_qkv(N, H, D, seed=0)
    out = torch.empty((N, H, D), dtype=torch.bfloat16, pin_memory=True)
    rows = signature_and_random_rows(N, 1024, seed=3)
    oracle = {}
    SNAPSHOTS.clear()

    def reference(kv_chunk):
        if kv_chunk not in oracle:
            oracle[kv_chunk] = oracle_rows(q, k, v, rows, kv_chunk=kv_chunk)
        return oracle[kv_chunk]

    yield q, k, v, out, rows, reference
    del q, k, v, out, oracle
    release_host_memory()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("budget_gib", sorted(SWEEP))
def test_config3_524k_56h_pinned_dram_workspace_sweep(sweep_inputs, budget_gib):
    q, k, v, out, rows, reference = sweep_inputs
    print(f"[gpu case] config 3: {N} x {H} x {D} bf16, pinned DRAM -> pinned DRAM, {budget_gib} GiB workspace",
          flush=True)
    cu = torch.tensor([0, N], dtype=torch.int32)
    config = StreamingAttentionConfig(workspace_budget_bytes=budget_gib * 2**30, backend="hip")
    plan = build_plan(q_heads=H, kv_heads=H, head_dim=D, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=N, max_kv_tokens=N, config=config)
    assert plan.block_m == 128
    assert (plan.q_chunk_tokens, plan.kv_chunk_tokens, plan.q_passes) == SWEEP[budget_gib]
    assert plan.estimated_workspace_bytes <= budget_gib * 2**30
    runner = StreamingAttentionRunner(plan, config)
    out.fill_(float("nan"))
    lse = torch.full((H, N), float("nan"), dtype=torch.float32, device="cuda")
    stats = StreamingAttentionStats()
    try:
        runner(q, k, v, cu, cu, out=out, lse_out=lse, stats=stats)
        torch.cuda.synchronize()
    finally:
        runner.close()
    print(f"    step done: {stats.wall_seconds:.2f} s, {plan.q_passes} passes, "
          f"H2D {stats.h2d_bytes / 1e9:.1f} GB", flush=True)
    assert stats.h2d_bytes == N * H * D * 2 * (1 + 2 * plan.q_passes)
    assert stats.d2h_bytes == N * H * D * 2
    ref_o, ref_l = reference(plan.kv_chunk_tokens)
    idx = torch.from_numpy(rows)
    SNAPSHOTS[budget_gib] = (out[idx].clone(), lse[:, idx.cuda()].cpu())
    check_parity(out[idx].float().numpy(), lse[:, idx.cuda()].cpu().numpy(), ref_o, ref_l,
                 f"{budget_gib} GiB: {rows.size} rows x {H} heads")


# Budget (GiB) -> the head-group plan's (buffer sets, K/V heads per unit,
# transposed V): two sets of one head, V transposed at 2 GiB (1.03 GiB used);
# at 1 GiB the transposed copy no longer fits beside two sets.
HEAD_GROUPS = {1: (2, 1, False), 2: (2, 1, True)}


@pytest.mark.timeout(600)
@pytest.mark.parametrize("budget_gib", sorted(HEAD_GROUPS))
def test_config3_524k_56h_head_groups(sweep_inputs, budget_gib):
    q, k, v, out, rows, reference = sweep_inputs
    print(f"[gpu case] config 3 head groups: {N} x {H} x {D} bf16, pinned DRAM -> pinned DRAM, "
          f"{budget_gib} GiB workspace", flush=True)
    cu = torch.tensor([0, N], dtype=torch.int32)
    config = StreamingAttentionConfig(workspace_budget_bytes=budget_gib * 2**30, backend="hip",
                                      schedule="head_groups")
    plan = build_plan(q_heads=H, kv_heads=H, head_dim=D, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=N, max_kv_tokens=N, config=config)
    assert (plan.head_group_sets, plan.head_group_kv_heads, plan.head_group_vt_bytes > 0) == HEAD_GROUPS[budget_gib]
    assert plan.kv_chunk_tokens == SWEEP[budget_gib][1]
    assert plan.estimated_workspace_bytes <= budget_gib * 2**30
    runner = StreamingAttentionRunner(plan, config)
    out.fill_(float("nan"))
    lse = torch.full((H, N), float("nan"), dtype=torch.float32, device="cuda")
    stats = StreamingAttentionStats()
    try:
        runner(q, k, v, cu, cu, out=out, lse_out=lse, stats=stats)
        torch.cuda.synchronize()
    finally:
        runner.close()
    print(f"    step done: {stats.wall_seconds:.2f} s, {plan.head_group_units} units, "
          f"H2D {stats.h2d_bytes / 1e9:.1f} GB", flush=True)
    assert stats.h2d_bytes == N * H * D * 2 * 3
    assert stats.d2h_bytes == N * H * D * 2
    idx = torch.from_numpy(rows)
    o_rows, l_rows = out[idx], lse[:, idx.cuda()].cpu()
    if budget_gib in SNAPSHOTS:
        torch.testing.assert_close(o_rows, SNAPSHOTS[budget_gib][0], atol=0, rtol=0)
        torch.testing.assert_close(l_rows, SNAPSHOTS[budget_gib][1], atol=0, rtol=0)
    ref_o, ref_l = reference(plan.kv_chunk_tokens)
    check_parity(o_rows.float().numpy(), l_rows.numpy(), ref_o, ref_l,
                 f"head groups {budget_gib} GiB: {rows.size} rows x {H} heads")
