"""GPU parity of paged mode with INT8 K/V pages (kv_storage_dtype="int8").

Pages are quantized per page (64-token groups from the page start) by the
memory source or the store writer, cross PCIe as int8 rows plus per-row fp16
scales and are dequantized in the update kernel.  Checks:

* bit for bit against tensor mode run on K/V that the oracle quantized and
  dequantized page by page (the kernel's dequantization is the reference's
  rounding and the chunk boundaries are the tensor-mode ones);
* against the FP32 oracle on the unquantized inputs with the reference's INT8
  bound (tests/test_paged_triton.py:87-91: relative L2 < 0.03, cosine > 0.995).
"""

from __future__ import annotations

import itertools
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import chunked_attention, dequantize_int8_groups, quantize_int8_groups
from seqattn import (
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


def config_for(*, q_chunk, kv_chunk, page_target_bytes, cache_mib=8, pinned_mib=8, depth=2, direct_io=False):
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
        kv_storage_dtype="int8",
    )


def dequantized_by_page(x: torch.Tensor, pages) -> torch.Tensor:
    """K or V as the INT8 pages hold it: the oracle's quantizer per page, then
    the kernel's dequantization rounding (bf16)."""
    out = torch.empty_like(x)
    for page in pages:
        rows = x[page.token_start : page.token_stop]
        q8, scales = quantize_int8_groups(rows.view(torch.int16).numpy().view(np.uint16))
        bits = dequantize_int8_groups(q8, scales)
        out[page.token_start : page.token_stop] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    return out


def tensor_mode(q, k, v, cu_q, cu_k, *, q_chunk, kv_chunk, causal):
    config = StreamingAttentionConfig(backend="hip", q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk)
    plan = build_plan(q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=q.shape[2], dtype=q.dtype, device="cuda",
                      max_q_tokens=q.shape[0], max_kv_tokens=k.shape[0], config=config)
    runner = StreamingAttentionRunner(plan, config)
    out = runner(q.pin_memory(), k.pin_memory(), v.pin_memory(), cu_q, cu_k, causal=causal)
    runner.close()
    return out


def reference_bound_check(out, q, k, v, cu_q, cu_k, *, q_chunk, kv_chunk, causal):
    ref, _ = chunked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q.numpy(),
                               cu_k.numpy(), q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk, causal=causal)
    got = out.float().numpy().reshape(-1)
    ref = ref.reshape(-1)
    rel_l2 = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    cosine = float(np.dot(got, ref) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    print(f"    vs unquantized oracle: relL2={rel_l2:.3e} cosine={cosine:.6f}", flush=True)
    assert rel_l2 < 0.03 and cosine > 0.995


@pytest.mark.parametrize("q_heads,kv_heads", [(8, 2), (4, 4)])
def test_int8_pages_at_reference_shapes(q_heads, kv_heads):
    """Reference tests/test_paged_triton.py:21-92 with storage_dtype="int8"."""
    announce(f"paged int8 reference shapes heads={q_heads}/{kv_heads}")
    torch.manual_seed(401)
    q = torch.randn(73, q_heads, 32, dtype=torch.bfloat16)
    k = torch.randn(89, kv_heads, 32, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    cu_q, cu_k = bounds([31, 0, 42]), bounds([37, 0, 52])
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, page_target_bytes=4096,
                              block_n=16, kv_storage_dtype="int8")
    config = config_for(q_chunk=23, kv_chunk=32, page_target_bytes=4096)
    out = torch.empty_like(q)
    stats = PagedAttentionStats()
    PagedAttentionRunner(config, device="cuda").run(source, source, cu_q, cu_k, MemoryPageSink(out), causal=True,
                                                    stats=stats)
    reference_bound_check(out, q, k, v, cu_q, cu_k, q_chunk=23, kv_chunk=32, causal=True)
    k_deq, v_deq = dequantized_by_page(k, source.kv_pages), dequantized_by_page(v, source.kv_pages)
    expected = tensor_mode(q, k_deq, v_deq, cu_q, cu_k, q_chunk=23, kv_chunk=32, causal=True)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    assert stats.kv_storage_dtype == "int8"
    assert stats.quantization_seconds > 0
    assert stats.operator_host_peak_bytes <= config.host_memory_budget_bytes


def test_int8_pages_gathered_into_chunks_gqa_d64():
    """64-token pages of a 1,500-key, two-segment causal GQA case gathered four
    at a time into 256-key launches."""
    announce("paged int8 gathered chunks d64")
    g = torch.Generator().manual_seed(9)
    q = torch.randn((1200, 8, 64), generator=g).to(torch.bfloat16)
    k = torch.randn((1500, 2, 64), generator=g)
    k[torch.randperm(1500, generator=g)[:15]] *= 8
    k = k.to(torch.bfloat16)
    v = torch.randn((1500, 2, 64), generator=g).to(torch.bfloat16)
    cu_q, cu_k = bounds([500, 700]), bounds([600, 900])
    page_bytes = 64 * 2 * 64 * 2
    source = MemoryPageSource(q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, page_target_bytes=page_bytes,
                              block_n=64, kv_storage_dtype="int8")
    config = config_for(q_chunk=384, kv_chunk=256, page_target_bytes=page_bytes)
    out = torch.empty_like(q)
    PagedAttentionRunner(config).run(source, source, cu_q, cu_k, MemoryPageSink(out), causal=True)
    k_deq, v_deq = dequantized_by_page(k, source.kv_pages), dequantized_by_page(v, source.kv_pages)
    expected = tensor_mode(q, k_deq, v_deq, cu_q, cu_k, q_chunk=384, kv_chunk=256, causal=True)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    reference_bound_check(out, q, k, v, cu_q, cu_k, q_chunk=384, kv_chunk=256, causal=True)


@pytest.mark.parametrize("direct_io", [False, True])
def test_int8_store_with_rolling_cache(tmp_path, direct_io):
    announce(f"paged int8 store, rolling cache, direct_io={direct_io}")
    g = torch.Generator().manual_seed(11)
    q = torch.randn((2048, 4, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((2048, 4, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((2048, 4, 128), generator=g).to(torch.bfloat16)
    cu = bounds([2048])
    page_bytes = 128 * 4 * 128  # 128-token pages of int8 rows
    try:
        store = NvmeQKVWriter.from_tensors(tmp_path / "store", q, k, v, cu, cu, page_target_bytes=page_bytes,
                                           block_n=64, kv_storage_dtype="int8", direct_io=direct_io)
    except RuntimeError as error:
        pytest.skip(f"no O_DIRECT support here: {error}")
    config = config_for(q_chunk=512, kv_chunk=512, page_target_bytes=page_bytes, cache_mib=1, depth=3,
                        direct_io=direct_io)
    # About six INT8 record slots (4 hot + 2 rolling) for 16 pages; 4 Q blocks re-scan K/V.
    config = replace(config, host_memory_budget_bytes=6 * 140 * 1024 + 13 * 2**20, cache_hot_fraction=0.7)
    out = torch.empty_like(q)
    stats = PagedAttentionStats()
    PagedAttentionRunner(config).run(store, store, cu, cu, MemoryPageSink(out), stats=stats)
    k_deq, v_deq = dequantized_by_page(k, store.kv_pages), dequantized_by_page(v, store.kv_pages)
    expected = tensor_mode(q, k_deq, v_deq, cu, cu, q_chunk=512, kv_chunk=512, causal=False)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    assert len(store.kv_pages) == 16 and stats.kv_pages == 4 * 16
    assert stats.cache_hits > 0 and stats.cache_misses > 16
    # int8 rows + per-row scales: about half the bf16 K/V bytes per page scanned.
    kv_bf16 = 4 * 2 * 2048 * 4 * 128 * 2
    assert stats.h2d_bytes < 0.6 * kv_bf16 + 4 * q.numel() * 2
    assert stats.operator_host_peak_bytes <= config.host_memory_budget_bytes
