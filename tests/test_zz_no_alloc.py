"""The allocation-free resident entry point against the existing one.

sa_run_resident_noalloc (its transposed V in the library's fixed device
array) must equal sa_pipeline_run_resident with caller-attached scratch
(reached through StreamingAttentionRunner with HBM-resident inputs) bit for
bit, output and LSE, on two calls in a row, the second with smaller inputs:
the array keeps the first call's contents, and the second call must neither
read them nor depend on them.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from seqattn import StreamingAttentionConfig, StreamingAttentionRunner, StreamingAttentionStats, _native, build_plan

pytestmark = pytest.mark.gpu


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)


def inputs(q_lengths, k_lengths, q_heads, kv_heads, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    nq, nk = sum(q_lengths), sum(k_lengths)
    q = (torch.randn((nq, q_heads, 128), generator=gen) * 1.3).to(dtype).cuda()
    k = torch.randn((nk, kv_heads, 128), generator=gen)
    k[torch.randperm(nk, generator=gen)[: max(1, nk // 100)]] *= 8  # 1% of key rows x8
    k = k.to(dtype).cuda()
    v = torch.randn((nk, kv_heads, 128), generator=gen).to(dtype).cuda()
    cu_q = torch.tensor([0, *torch.tensor(q_lengths).cumsum(0).tolist()], dtype=torch.int32)
    cu_k = torch.tensor([0, *torch.tensor(k_lengths).cumsum(0).tolist()], dtype=torch.int32)
    return q, k, v, cu_q, cu_k


def existing_entry_point(q, k, v, cu_q, cu_k, *, kv_chunk, causal, scale):
    config = StreamingAttentionConfig(backend="hip", kv_chunk_tokens=kv_chunk)
    plan = build_plan(q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=128, dtype=q.dtype, device="cuda",
                      max_q_tokens=q.shape[0], max_kv_tokens=k.shape[0], config=config)
    runner = StreamingAttentionRunner(plan, config)
    stats = StreamingAttentionStats()
    out, lse = runner(q, k, v, cu_q, cu_k, causal=causal, softmax_scale=scale, return_lse=True, stats=stats)
    torch.cuda.synchronize()
    runner.close()
    assert stats.resident_scratch_bytes > 0, "the existing path did not read V through its transposed copy"
    return out, lse


def noalloc_entry_point(q, k, v, cu_q, cu_k, *, kv_chunk, causal, scale):
    lib = _native.lib()
    out = torch.full_like(q, float("nan"))
    lse = torch.full((q.shape[1], q.shape[0]), float("nan"), dtype=torch.float32, device="cuda")
    bounds_q = (ctypes.c_int64 * cu_q.numel())(*cu_q.tolist())
    bounds_k = (ctypes.c_int64 * cu_k.numel())(*cu_k.tolist())
    status = lib.sa_run_resident_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1), out.stride(0), out.stride(1),
        lse.stride(0), bounds_q, bounds_k, cu_q.numel() - 1, q.shape[1], k.shape[1], 128,
        _native.dtype_code(q.dtype), kv_chunk, scale, int(causal), torch.cuda.current_stream().cuda_stream)
    _native.check(status, "sa_run_resident_noalloc")
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_noalloc_equals_the_attached_scratch_path_on_two_calls(dtype, causal):
    calls = [
        # (q segment lengths, k segment lengths, heads, K/V chunk): the second call is smaller
        ([3000, 0, 1700], [4100, 300, 2500], (8, 2), 1024),
        ([700], [900], (4, 4), 512),
    ]
    for index, (q_lengths, k_lengths, (q_heads, kv_heads), kv_chunk) in enumerate(calls):
        announce(f"no-alloc call {index + 1}: {dtype} causal={causal} q={q_lengths} k={k_lengths}")
        q, k, v, cu_q, cu_k = inputs(q_lengths, k_lengths, q_heads, kv_heads, dtype, seed=40 + index)
        ref_out, ref_lse = existing_entry_point(q, k, v, cu_q, cu_k, kv_chunk=kv_chunk, causal=causal, scale=0.09)
        out, lse = noalloc_entry_point(q, k, v, cu_q, cu_k, kv_chunk=kv_chunk, causal=causal, scale=0.09)
        assert torch.equal(out, ref_out)
        assert torch.equal(lse, ref_lse)


def test_noalloc_rejects_a_segment_beyond_its_scratch():
    announce("no-alloc rejects an oversized segment")
    q = torch.zeros((4, 2, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((131_073, 2, 128), dtype=torch.bfloat16, device="cuda")
    lib = _native.lib()
    status = lib.sa_run_resident_noalloc(
        q.data_ptr(), k.data_ptr(), k.data_ptr(), q.data_ptr(), None, 256, 128, 256, 128, 256, 128, 256, 128, 0,
        (ctypes.c_int64 * 2)(0, 4), (ctypes.c_int64 * 2)(0, 131_073), 1, 2, 2, 128, 0, 1024, 0.1, 0,
        torch.cuda.current_stream().cuda_stream)
    assert status == -1
    assert b"needs 67141632 bytes" in lib.sa_last_error()
