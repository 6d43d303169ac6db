"""GPU parity of paged mode (the native pipeline fed from page sources).

Against the CPU oracle at the reference's paged test shapes
(tests/test_paged_triton.py:22-93: bf16 relative L2 < 0.005, max-abs <=
0.015625) and, bit for bit, against tensor mode on the same inputs: paged
mode gathers K/V pages into the same kv_chunk-aligned launches, and each
query's result does not depend on the Q block it lands in.
"""

from __future__ import annotations

import itertools
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import chunked_attention
from seqattn import (
    CallbackOutputSink,
    MemoryPageSink,
    MemoryPageSource,
    NvmeQKVWriter,
    PagedAttentionConfig,
    PagedAttentionRunner,
    PagedAttentionStats,
    StreamingAttentionConfig,
    StreamingAttentionRunner,
    build_plan,
)

pytestmark = pytest.mark.gpu


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)


def bounds(lengths):
    return torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32)


def paged_config(*, q_chunk, kv_chunk, page_target_bytes, cache_mib=8, pinned_mib=8, depth=2,
                 storage="bf16", direct_io=False):
    return PagedAttentionConfig(
        attention=StreamingAttentionConfig(backend="hip", workspace_budget_bytes=256 * 2**20,
                                           q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk, num_output_buffers=2),
        host_memory_budget_bytes=(cache_mib + pinned_mib + 4 + 1) * 2**20,
        pinned_staging_budget_bytes=pinned_mib * 2**20,
        direct_io_bounce_budget_bytes=4 * 2**20,
        metadata_margin_bytes=1 * 2**20,
        page_target_bytes=page_target_bytes,
        io_workers=2,
        io_queue_depth=depth,
        num_output_buffers=2,
        direct_io=direct_io,
        kv_storage_dtype=storage,
    )


def tensor_mode(q, k, v, cu_q, cu_k, *, q_chunk, kv_chunk, causal):
    config = StreamingAttentionConfig(backend="hip", q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk)
    plan = build_plan(q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=q.shape[2], dtype=q.dtype, device="cuda",
                      max_q_tokens=q.shape[0], max_kv_tokens=k.shape[0], config=config)
    runner = StreamingAttentionRunner(plan, config)
    out, lse = runner(q.pin_memory(), k.pin_memory(), v.pin_memory(), cu_q, cu_k, causal=causal, return_lse=True)
    runner.close()
    return out, lse


def oracle_check(out, q, k, v, cu_q, cu_k, *, q_chunk, kv_chunk, causal, rows=None):
    ref, _ = chunked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q.numpy(),
                               cu_k.numpy(), q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk, causal=causal,
                               rows=rows)
    got = out.float().numpy()
    if rows is not None:
        got, ref = got[rows], ref[rows]
    diff = np.abs(got - ref)
    rel_l2 = float(np.linalg.norm(diff) / np.linalg.norm(ref))
    print(f"    max|dO|={diff.max():.3e} relL2={rel_l2:.3e}", flush=True)
    assert rel_l2 < 0.005
    assert diff.max() <= 0.015625


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(8, 2), (4, 4)])
def test_paged_matches_oracle_and_tensor_mode_at_reference_shapes(causal, q_heads, kv_heads):
    announce(f"paged reference shapes causal={causal} heads={q_heads}/{kv_heads}")
    torch.manual_seed(401)
    q = torch.randn(73, q_heads, 32, dtype=torch.bfloat16)
    k = torch.randn(89, kv_heads, 32, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    cu_q, cu_k = bounds([31, 0, 42]), bounds([37, 0, 52])
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, page_target_bytes=4096,
                              block_n=16)
    config = paged_config(q_chunk=23, kv_chunk=32, page_target_bytes=4096)
    out = torch.empty_like(q)
    stats = PagedAttentionStats()
    PagedAttentionRunner(config, device="cuda").run(source, source, cu_q, cu_k, MemoryPageSink(out),
                                                    causal=causal, stats=stats)
    oracle_check(out, q, k, v, cu_q, cu_k, q_chunk=23, kv_chunk=32, causal=causal)
    expected, _ = tensor_mode(q, k, v, cu_q, cu_k, q_chunk=23, kv_chunk=32, causal=causal)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    assert stats.operator_host_peak_bytes <= config.host_memory_budget_bytes
    assert stats.cache_hits + stats.cache_misses == stats.kv_pages
    assert stats.q_pages == len(source.q_pages)
    assert stats.backend == "hip"


def _inputs(n_q, n_k, q_heads, kv_heads, d, seed, outliers=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((n_q, q_heads, d), generator=g)
    k = torch.randn((n_k, kv_heads, d), generator=g)
    if outliers:
        idx = torch.randperm(n_k, generator=g)[: max(1, n_k // 100)]
        k[idx] *= 8
    v = torch.randn((n_k, kv_heads, d), generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("pinned", [False, True])
def test_memory_source_pinned_zero_copy_and_staged_paths_agree(pinned):
    announce(f"memory source pinned={pinned}")
    q, k, v = _inputs(1200, 1500, 8, 4, 128, 3)
    cu_q, cu_k = bounds([500, 700]), bounds([600, 900])
    if pinned:
        q, k, v = q.pin_memory(), k.pin_memory(), v.pin_memory()
    # 64-token pages (64 KiB per K page), kv_chunk 256 -> four pages per launch.
    page_bytes = 64 * 4 * 128 * 2
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                              page_target_bytes=page_bytes, block_n=64)
    config = paged_config(q_chunk=384, kv_chunk=256, page_target_bytes=page_bytes)
    out = torch.empty_like(q)
    if pinned:
        out = out.pin_memory()
    PagedAttentionRunner(config).run(source, source, cu_q, cu_k, MemoryPageSink(out), causal=True)
    expected, _ = tensor_mode(q, k, v, cu_q, cu_k, q_chunk=384, kv_chunk=256, causal=True)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    rows = np.arange(0, 1200, 7)
    oracle_check(out, q, k, v, cu_q, cu_k, q_chunk=384, kv_chunk=256, causal=True, rows=rows)


@pytest.mark.parametrize("direct_io", [False, True])
def test_nvme_store_with_rolling_cache_and_staging(tmp_path, direct_io):
    announce(f"nvme store, cache smaller than K/V, direct_io={direct_io}")
    q, k, v = _inputs(2048, 2048, 4, 4, 128, 11, outliers=True)
    cu = bounds([2048])
    page_bytes = 128 * 4 * 128 * 2  # 128-token pages, 256 KiB K+V records
    try:
        store = NvmeQKVWriter.from_tensors(tmp_path / "store", q, k, v, cu, cu, page_target_bytes=page_bytes,
                                           block_n=64, kv_storage_dtype="bf16", direct_io=direct_io)
    except RuntimeError as error:
        pytest.skip(f"no O_DIRECT support here: {error}")
    # 16 K/V pages; cache of 6 record slots (4 hot + 2 rolling); 4 Q blocks re-scan K/V.
    config = paged_config(q_chunk=512, kv_chunk=512, page_target_bytes=page_bytes, cache_mib=1, pinned_mib=8,
                          depth=3, direct_io=direct_io)
    config = replace(config, host_memory_budget_bytes=6 * 256 * 1024 + 13 * 2**20, cache_hot_fraction=0.7)
    out = torch.empty_like(q)
    stats = PagedAttentionStats()
    PagedAttentionRunner(config).run(store, store, cu, cu, MemoryPageSink(out), stats=stats)
    expected, expected_lse = tensor_mode(q, k, v, cu, cu, q_chunk=512, kv_chunk=512, causal=False)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    assert stats.kv_pages == 4 * 16
    assert stats.cache_hits > 0 and stats.cache_misses > 16
    assert stats.nvme_logical_read_bytes > 0
    assert stats.operator_host_peak_bytes <= config.host_memory_budget_bytes


def test_device_output_mode_and_lse_match_host_output(tmp_path):
    announce("paged device-consumer output")
    q, k, v = _inputs(1000, 1100, 8, 2, 128, 13, outliers=True)
    cu_q, cu_k = bounds([400, 600]), bounds([500, 600])
    page_bytes = 64 * 2 * 128 * 2
    store = NvmeQKVWriter.from_tensors(tmp_path / "s", q, k, v, cu_q, cu_k, page_target_bytes=page_bytes,
                                       block_n=64, direct_io=False)
    config = paged_config(q_chunk=256, kv_chunk=192, page_target_bytes=page_bytes)
    runner = PagedAttentionRunner(config)
    host = torch.empty_like(q)
    runner.run(store, store, cu_q, cu_k, MemoryPageSink(host), causal=True)
    lse = torch.empty((8, 1000), device="cuda")
    device_out = runner.run_with_device_output(store, store, cu_q, cu_k, causal=True, lse_out=lse)
    torch.cuda.synchronize()
    assert device_out.device.type == "cuda"
    torch.testing.assert_close(device_out.cpu(), host, atol=0, rtol=0)
    expected, expected_lse = tensor_mode(q, k, v, cu_q, cu_k, q_chunk=256, kv_chunk=192, causal=True)
    torch.testing.assert_close(host, expected, atol=0, rtol=0)
    torch.testing.assert_close(lse.cpu(), expected_lse, atol=0, rtol=0)
    doubled = runner.run_with_device_output(store, store, cu_q, cu_k, causal=True,
                                            out=torch.empty((1000, 8 * 128), dtype=torch.bfloat16, device="cuda"),
                                            output_transform=lambda tile, s, e: tile * 2)
    torch.cuda.synchronize()
    torch.testing.assert_close(doubled.cpu(), (expected.reshape(1000, -1).float() * 2).to(torch.bfloat16),
                               atol=0, rtol=0)


def test_callback_sink_reuses_bounded_output_ring():
    announce("callback sink ring")
    torch.manual_seed(223)
    q = torch.randn(97, 4, 16, dtype=torch.bfloat16)
    k = torch.randn(97, 2, 16, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    cu = bounds([97])
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu, cu_seqlens_k=cu, page_target_bytes=2048, block_n=16)
    pages, storages = [], set()

    def consume(page, data):
        pages.append((page, data.clone()))
        storages.add(data.untyped_storage().data_ptr())

    result = PagedAttentionRunner(paged_config(q_chunk=7, kv_chunk=16, page_target_bytes=2048)).run(
        source, source, cu, cu, CallbackOutputSink(consume))
    assert result == len(source.q_pages)
    assert len(storages) <= 2
    assembled = torch.empty_like(q)
    for page, data in pages:
        assembled[page.token_start : page.token_stop].copy_(data)
    oracle_check(assembled, q, k, v, cu, cu, q_chunk=7, kv_chunk=16, causal=False)


def test_tiny_pinned_budget_forces_early_flushes_and_stays_exact():
    announce("stage ring pressure")
    q, k, v = _inputs(600, 900, 4, 4, 64, 17)
    cu = bounds([900 - 300, 300])
    cu_q = bounds([300, 300])
    page_bytes = 32 * 4 * 64 * 2
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu, page_target_bytes=page_bytes,
                              block_n=32)
    # Pinned budget: a few 32 KiB stage slots and small Q / output staging.
    config = paged_config(q_chunk=512, kv_chunk=512, page_target_bytes=page_bytes, pinned_mib=1)
    config = replace(config, pinned_staging_budget_bytes=320 * 1024)
    out = torch.empty_like(q)
    PagedAttentionRunner(config).run(source, source, cu_q, cu, MemoryPageSink(out), causal=True)
    oracle_check(out, q, k, v, cu_q, cu, q_chunk=512, kv_chunk=512, causal=True)
