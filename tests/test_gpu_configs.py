"""GPU parity at every workload the benchmark configuration names, O and LSE.

Each case runs the product path (libseqattn_hip.so through the seqattn API)
on the configuration's own shape and seeded inputs and compares the output
and the natural-log LSE with the CPU oracle: all rows for the 4,096-token
case, and for the long sequences (the 524,288-token workspace sweep is in
test_gpu_config3_sweep.py) the reference's large-tier signature rows
{0, N/4, N/2, 3N/4, N-1} (benchmarks/large_tier_comparison.py:62-66) plus
1,024 seeded-random rows, every head, against every key.  Tolerances: O
max-abs <= 2e-2, LSE max-abs <= 1e-3, O relative L2 <= 5e-3, every element
within 2^-5 (|ref| + rms(ref)).
"""

from __future__ import annotations

import os
import tempfile
import warnings
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import chunked_attention, dense_attention_f64
from seqattn import (
    NvmeQKVWriter,
    PagedAttentionConfig,
    PagedAttentionRunner,
    PagedAttentionStats,
    StreamingAttentionConfig,
    StreamingAttentionRunner,
    StreamingAttentionStats,
    build_plan,
    ephemeral_nvme_directory,
    streaming_attn_func,
    streaming_attn_varlen_func,
)
from seeded import (
    RunModeNotice,
    check_parity,
    oracle_rows,
    release_host_memory,
    seeded_qkv,
    signature_and_random_rows,
)

pytestmark = pytest.mark.gpu


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)


@pytest.fixture(autouse=True)
def _free_pinned_memory():
    yield
    release_host_memory()


def test_config1_4096x8x64_all_rows_on_the_hip_path():
    # Config 1's shape and inputs: fp32 Q, K, V ~ N(0,1) drawn in that order
    # from one generator seeded 0; query block 1,024, K/V chunk 512.  The HIP
    # path computes in bf16, so the fp32 draws are rounded to bf16 first and
    # the oracle sees the same bf16 values.
    announce("config 1: 4,096 x 8 x 64, q block 1,024, kv chunk 512")
    gen = torch.Generator().manual_seed(0)
    shape = (4096, 8, 64)
    q, k, v = (torch.randn(shape, generator=gen).to(torch.bfloat16).pin_memory() for _ in range(3))
    cu = torch.tensor([0, 4096], dtype=torch.int32)
    config = StreamingAttentionConfig(backend="hip", q_chunk_tokens=1024, kv_chunk_tokens=512)
    plan = build_plan(q_heads=8, kv_heads=8, head_dim=64, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=4096, max_kv_tokens=4096, config=config)
    runner = StreamingAttentionRunner(plan, config)
    out, lse = runner(q, k, v, cu, cu, return_lse=True)
    runner.close()
    ref_o, ref_l = chunked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), [0, 4096], [0, 4096],
                                     q_chunk_tokens=1024, kv_chunk_tokens=512)
    check_parity(out.float().numpy(), lse.numpy(), ref_o, ref_l, "vs oracle")
    # and against the dense float64 closed form softmax(QK^T / sqrt(d)) V
    dense_o, dense_l = dense_attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                           [0, 4096], [0, 4096])
    check_parity(out.float().numpy(), lse.numpy(), dense_o.astype(np.float32), dense_l.astype(np.float32),
                 "vs dense f64")


@pytest.mark.timeout(900)
def test_config4_paged_158k_48h_256_token_pages_from_an_aligned_store():
    n, h, d, page_tokens = 158_208, 48, 128, 256
    announce(f"config 4: paged {n} x {h} x {d}, {page_tokens}-token pages, O_DIRECT store, 16 GiB cache")
    q, k, v = seeded_qkv(n, h, d, seed=0, pinned=False)
    outliers = torch.from_numpy(np.sort(np.random.default_rng(7).choice(n, n // 100, replace=False)))
    k[outliers] *= 8  # 1% of key rows x8 (exact in bf16)
    cu = torch.tensor([0, n], dtype=torch.int32)
    page_bytes = page_tokens * h * d * 2
    parent = Path(os.environ.get("TMPDIR", tempfile.gettempdir()))
    with ephemeral_nvme_directory(parent) as root:
        try:
            store = NvmeQKVWriter.from_tensors(root / "qkv", q, k, v, cu, cu, page_target_bytes=page_bytes,
                                               block_n=64, direct_io=True)
            direct_io = True
            refused = ""
        except RuntimeError as error:
            # A filesystem without O_DIRECT (tmpfs): the same records, buffered.
            refused = f"{error}"
            store = NvmeQKVWriter.from_tensors(root / "qkv-buffered", q, k, v, cu, cu,
                                               page_target_bytes=page_bytes, block_n=64, direct_io=False)
            direct_io = False
        assert len(store.kv_pages) == n // page_tokens
        config = PagedAttentionConfig(
            attention=StreamingAttentionConfig(workspace_budget_bytes=2 * 2**30, backend="hip"),
            host_memory_budget_bytes=16 * 2**30 + 2**30 + 512 * 2**20 + 128 * 2**20,
            page_target_bytes=page_bytes,
            io_queue_depth=4,
            direct_io=direct_io,
        )
        runner = PagedAttentionRunner(config)
        out = torch.empty((n, h, d), dtype=torch.bfloat16, device="cuda")
        lse = torch.empty((h, n), dtype=torch.float32, device="cuda")
        stats = PagedAttentionStats()
        runner.run_with_device_output(store, store, cu, cu, out=out, lse_out=lse, stats=stats)
        torch.cuda.synchronize()
    warnings.warn(RunModeNotice(
        f"config 4 read its pages from an O_DIRECT store under {parent}" if direct_io else
        f"config 4 read its pages from a BUFFERED store under {parent}: O_DIRECT was refused ({refused})"))
    print(f"    direct_io={direct_io} cache hit ratio {stats.cache_hit_ratio:.3f} "
          f"q chunks {stats.q_chunks} kv pages {stats.kv_pages}", flush=True)
    rows = signature_and_random_rows(n, 1024, seed=4)
    ref_o, ref_l = oracle_rows(q, k, v, rows, kv_chunk=8192)
    idx = torch.from_numpy(rows).cuda()
    check_parity(out[idx].float().cpu().numpy(), lse[:, idx].cpu().numpy(), ref_o, ref_l,
                 f"{rows.size} rows x {h} heads")


@pytest.mark.timeout(1200)
def test_config5_1m_64h_peaked_keys_8gib_workspace():
    n, h, d = 1_048_576, 64, 128
    announce(f"config 5: {n} x {h} x {d}, K scaled per head by U[0.5, 4], 8 GiB workspace, kv chunk 8,192")
    head_scale = np.random.default_rng(11).uniform(0.5, 4.0, size=h).astype(np.float32)
    q, k, v = seeded_qkv(n, h, d, seed=0, k_head_scale=head_scale)
    cu = torch.tensor([0, n], dtype=torch.int32)
    # Q/K/V (48 GiB) are page-locked.  Where the host refuses to page-lock a
    # fourth 16 GiB buffer for the output (MI355X boxes here stop between 48
    # and 64 GiB of page-locked memory), the output is pageable host memory,
    # which the runner accepts with pin_output=False (its D2H copies then go
    # through the runtime's staging).
    try:
        out = torch.empty((n, h, d), dtype=torch.bfloat16, pin_memory=True)
    except RuntimeError as error:
        refused = f"{type(error).__name__}: {error}"
        out = torch.empty((n, h, d), dtype=torch.bfloat16)
    warnings.warn(RunModeNotice(
        "config 5 wrote its output to page-locked host memory" if out.is_pinned() else
        f"config 5 wrote its output to PAGEABLE host memory (page-locking 16 GiB failed: {refused}); the Q-block "
        "run's copies went through the runtime's staging, the head-group run's through the pipeline's page-locked "
        "staging"))
    config = StreamingAttentionConfig(workspace_budget_bytes=8 * 2**30, kv_chunk_tokens=8192, backend="hip",
                                      pin_output=out.is_pinned())
    plan = build_plan(q_heads=h, kv_heads=h, head_dim=d, dtype=torch.bfloat16, device="cuda",
                      max_q_tokens=n, max_kv_tokens=n, config=config)
    runner = StreamingAttentionRunner(plan, config)
    lse = torch.empty((h, n), dtype=torch.float32, device="cuda")
    stats = StreamingAttentionStats()
    runner(q, k, v, cu, cu, out=out, lse_out=lse, stats=stats)
    torch.cuda.synchronize()
    runner.close()
    print(f"    step done: {stats.wall_seconds:.2f} s, {plan.q_passes} passes, "
          f"H2D {stats.h2d_bytes / 1e9:.1f} GB", flush=True)
    rows = signature_and_random_rows(n, 1024, seed=5)
    ref_o, ref_l = oracle_rows(q, k, v, rows, kv_chunk=8192)
    idx = torch.from_numpy(rows)
    o_rows, l_rows = out[idx].clone(), lse[:, idx.cuda()].cpu()
    check_parity(o_rows.float().numpy(), l_rows.numpy(), ref_o, ref_l, f"{rows.size} rows x {h} heads")
    # The same step in the head-group schedule (24 units of up to 3 K/V heads; a
    # pageable output goes through the pipeline's page-locked staging):
    # the same bits on the sampled rows.
    hg_config = StreamingAttentionConfig(workspace_budget_bytes=8 * 2**30, kv_chunk_tokens=8192, backend="hip",
                                         pin_output=out.is_pinned(), schedule="head_groups")
    hg_plan = build_plan(q_heads=h, kv_heads=h, head_dim=d, dtype=torch.bfloat16, device="cuda",
                         max_q_tokens=n, max_kv_tokens=n, config=hg_config)
    assert (hg_plan.head_group_sets, hg_plan.head_group_kv_heads, hg_plan.head_group_units) == (2, 3, 24)
    runner = StreamingAttentionRunner(hg_plan, hg_config)
    out.fill_(float("nan"))
    lse.fill_(float("nan"))
    hg_stats = StreamingAttentionStats()
    try:
        runner(q, k, v, cu, cu, out=out, lse_out=lse, stats=hg_stats)
        torch.cuda.synchronize()
    finally:
        runner.close()
    print(f"    head groups: {hg_stats.wall_seconds:.2f} s, H2D {hg_stats.h2d_bytes / 1e9:.1f} GB", flush=True)
    assert hg_stats.h2d_bytes == 3 * n * h * d * 2
    torch.testing.assert_close(out[idx], o_rows, atol=0, rtol=0)
    torch.testing.assert_close(lse[:, idx.cuda()].cpu(), l_rows, atol=0, rtol=0)


@pytest.mark.parametrize("schedule", ["q_blocks", "head_groups"])
@pytest.mark.parametrize("causal", [True, False])
def test_dense_and_varlen_api_wrappers_on_the_hip_path(causal, schedule):
    # The reference's tests/test_api.py:7-25 shapes (batch 2, 7 queries,
    # 9 keys, 4 query heads over 2 K/V heads, d 32, q chunk 3, kv chunk 4),
    # in bf16 on the HIP path, against the oracle; in both schedules.
    announce(f"API wrappers causal={causal} schedule={schedule}")
    torch.manual_seed(11)
    q = torch.randn(2, 7, 4, 32).to(torch.bfloat16)
    k = torch.randn(2, 9, 2, 32).to(torch.bfloat16)
    v = torch.randn_like(k.float()).to(torch.bfloat16)
    config = StreamingAttentionConfig(backend="hip", q_chunk_tokens=3, kv_chunk_tokens=4, schedule=schedule)
    dense = streaming_attn_func(q.pin_memory(), k.pin_memory(), v.pin_memory(), causal=causal, config=config)
    assert dense.shape == q.shape and dense.dtype == q.dtype and dense.device.type == "cpu"
    cu_q = torch.tensor([0, 7, 14], dtype=torch.int32)
    cu_k = torch.tensor([0, 9, 18], dtype=torch.int32)
    packed_q, packed_k, packed_v = (t.reshape(-1, t.shape[2], t.shape[3]).pin_memory() for t in (q, k, v))
    varlen, lse = streaming_attn_varlen_func(packed_q, packed_k, packed_v, cu_q, cu_k, 7, 9, causal=causal,
                                             config=config, return_lse=True)
    assert torch.equal(varlen.reshape_as(dense), dense)
    ref_o, ref_l = chunked_attention(packed_q.float().numpy(), packed_k.float().numpy(), packed_v.float().numpy(),
                                     cu_q.numpy(), cu_k.numpy(), q_chunk_tokens=3, kv_chunk_tokens=4, causal=causal)
    check_parity(varlen.float().numpy(), lse.numpy(), ref_o, ref_l, "varlen")
    with pytest.raises(ValueError, match="cu_seqlens_q exceeds max_seqlen_q"):
        streaming_attn_varlen_func(packed_q, packed_k, packed_v, cu_q, cu_k, 6, 9, config=config)
