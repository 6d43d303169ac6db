"""GPU parity of the projected pipeline (hidden -> QKV -> streamed attention ->
output projection) against the CPU oracle.

Follows the reference's tests/test_pipeline.py:23-190 (same shapes, chunking
and stats assertions) for both Q/K/V residencies.  The expected output is
built from the Q/K/V the caller's projection produces (the same per-chunk
GEMMs, so the same bits), the FP32 oracle attention rounded to the input
dtype as the finalize step does, and the output projection in float64 on
the CPU.  Tolerances: the reference's assert_close bound (atol 7e-2,
rtol 1e-2), relative L2 <= 1e-2, and every element within
2^-5 * (|ref| + rms(ref)).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import chunked_attention
from seqattn import (
    ProjectedAttentionRunner,
    ProjectedAttentionStats,
    ProjectionPipelineConfig,
    StreamingAttentionConfig,
    build_plan,
    streaming_projected_self_attention,
)

pytestmark = pytest.mark.gpu


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)


class Projections:
    """Bias-free QKV and output projections with seeded weights."""

    def __init__(self, hidden, q_heads, kv_heads, head_dim, out_features, dtype, seed):
        gen = torch.Generator().manual_seed(seed)
        self.q_heads, self.kv_heads, self.head_dim = q_heads, kv_heads, head_dim
        inner_q, inner_kv = q_heads * head_dim, kv_heads * head_dim
        self.w_qkv_cpu = (torch.randn(inner_q + 2 * inner_kv, hidden, generator=gen) * hidden**-0.5).to(dtype)
        self.w_out_cpu = (torch.randn(out_features, inner_q, generator=gen) * inner_q**-0.5).to(dtype)
        self.w_qkv = self.w_qkv_cpu.cuda()
        self.w_out = self.w_out_cpu.cuda()
        self.qkv_calls: list[tuple[int, int]] = []
        self.out_calls: list[tuple[int, int]] = []

    def project_qkv(self, hidden, start, stop):
        self.qkv_calls.append((start, stop))
        qkv = hidden @ self.w_qkv.t()
        n = hidden.shape[0]
        q_end = self.q_heads * self.head_dim
        kv = self.kv_heads * self.head_dim
        q = qkv[:, :q_end].reshape(n, self.q_heads, self.head_dim).contiguous()
        k = qkv[:, q_end:q_end + kv].reshape(n, self.kv_heads, self.head_dim).contiguous()
        v = qkv[:, q_end + kv:].reshape(n, self.kv_heads, self.head_dim).contiguous()
        return q, k, v

    def output_projector(self, attention, start, stop):
        self.out_calls.append((start, stop))
        return attention @ self.w_out.t()

    def expected(self, hidden_cpu, cu, *, projection_chunk, q_chunk, kv_chunk, causal, dtype):
        """Per-chunk GPU projection (same GEMM shapes as the runner), FP32
        oracle attention rounded to ``dtype``, float64 output projection."""
        parts = [
            self.project_qkv(hidden_cpu[s:s + projection_chunk].cuda(), s, 0)
            for s in range(0, hidden_cpu.shape[0], projection_chunk)
        ]
        q, k, v = (torch.cat([p[i] for p in parts]).cpu() for i in range(3))
        self.qkv_calls.clear()
        o, _ = chunked_attention(
            q.float().numpy(), k.float().numpy(), v.float().numpy(), np.asarray(cu), np.asarray(cu),
            q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk, causal=causal,
        )
        attention = torch.from_numpy(o).to(dtype).double().reshape(o.shape[0], -1)
        return (attention @ self.w_out_cpu.double().t()).numpy(), (q, k, v)


def check_projected(actual: torch.Tensor, expected: np.ndarray) -> None:
    a = actual.double().numpy()
    assert np.isfinite(a).all()
    torch.testing.assert_close(torch.from_numpy(a), torch.from_numpy(expected), atol=7e-2, rtol=1e-2)
    diff = np.abs(a - expected)
    norm = float(np.sqrt(np.square(expected).sum()))
    rel_l2 = float(np.sqrt(np.square(diff).sum())) / norm if norm else 0.0
    rms = math.sqrt(float(np.square(expected).mean())) if expected.size else 0.0
    scaled = float((diff / (np.abs(expected) + rms)).max()) if expected.size else 0.0
    print(f"  max|d| {diff.max() if diff.size else 0:.3e} relL2 {rel_l2:.3e} scaled {scaled:.3e}", flush=True)
    assert rel_l2 <= 1e-2
    assert scaled <= 2.0**-5


def run_pipeline(residency, dtype, *, tokens, hidden, heads, kv_heads, head_dim, cu, attention_config,
                 projection_chunk, causal=False, seed=101, buffers=2):
    torch.manual_seed(seed)
    hidden_cpu = torch.randn(tokens, hidden, generator=torch.Generator().manual_seed(seed)).to(dtype).pin_memory()
    proj = Projections(hidden, heads, kv_heads, head_dim, hidden, dtype, seed + 1)
    pipeline_config = ProjectionPipelineConfig(
        projection_chunk_tokens=projection_chunk, num_projection_buffers=buffers, qkv_residency=residency
    )
    plan = build_plan(
        q_heads=heads, kv_heads=kv_heads, head_dim=head_dim, dtype=dtype, device="cuda",
        max_q_tokens=tokens, max_kv_tokens=tokens, config=attention_config,
    )
    runner = ProjectedAttentionRunner(plan, attention_config, pipeline_config)
    stats = ProjectedAttentionStats()
    actual = runner(
        hidden_cpu, cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector,
        output_features=hidden, causal=causal, stats=stats,
    )
    torch.cuda.synchronize()
    return runner, proj, hidden_cpu, actual, stats


REFERENCE_ATTENTION = dict(q_chunk_tokens=41, kv_chunk_tokens=29, block_m=16, block_n=16, num_output_buffers=2)


@pytest.mark.parametrize("residency", ["host", "hbm"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_projected_pipeline_matches_oracle(dtype, residency):
    """Reference test_pipeline.py:23-114: 97 tokens, hidden 48, 4 heads x 16,
    segments [0, 37, 37, 97] (an empty middle one), Q chunk 41, K/V chunk 29,
    projection chunk 31."""
    announce(f"projected 97 tokens {dtype} {residency}")
    tokens, hidden, heads, head_dim = 97, 48, 4, 16
    inner = heads * head_dim
    cu = torch.tensor([0, 37, 37, 97], dtype=torch.int32)
    config = StreamingAttentionConfig(backend="triton", **REFERENCE_ATTENTION)
    runner, proj, hidden_cpu, actual, stats = run_pipeline(
        residency, dtype, tokens=tokens, hidden=hidden, heads=heads, kv_heads=heads, head_dim=head_dim,
        cu=cu, attention_config=config, projection_chunk=31,
    )
    assert proj.qkv_calls == [(0, 31), (31, 62), (62, 93), (93, 97)]
    # Output tiles are segment-bounded Q chunks of the planned size (41 aligned
    # down to block_m 16), as the streamed runner hands them out.
    assert runner.plan.q_chunk_tokens == 32
    assert proj.out_calls == [(0, 32), (32, 37), (37, 69), (69, 97)]
    expected, _ = proj.expected(hidden_cpu, cu.tolist(), projection_chunk=31, q_chunk=41, kv_chunk=29,
                                causal=False, dtype=dtype)
    check_projected(actual, expected)
    element = actual.element_size()
    assert stats.projection_chunks == math.ceil(tokens / 31)
    assert stats.attention.d2h_bytes == tokens * hidden * element
    assert stats.raw_attention_roundtrip_bytes_avoided == 2 * tokens * inner * element
    assert stats.projection_hidden_h2d_bytes == tokens * hidden * element
    if residency == "host":
        assert stats.projection_qkv_d2h_bytes == 3 * tokens * inner * element
        assert stats.qkv_host_bytes == 3 * tokens * inner * element
    else:
        assert stats.projection_qkv_d2h_bytes == 0
        assert stats.attention.h2d_bytes == 0
    assert stats.as_dict()["total_d2h_bytes"] == stats.projection_qkv_d2h_bytes + stats.attention.d2h_bytes


@pytest.mark.parametrize("causal", [False, True])
def test_hbm_residency_is_bit_identical_to_host_residency(causal):
    """GQA (8 query heads over 2 K/V heads), head_dim 64, two segments, a
    Q chunk that splits a segment: both residencies run the same kernels on
    the same chunk schedule and the same output-projection tiles."""
    announce(f"projected 3000 tokens GQA causal={causal} host vs hbm")
    kwargs = dict(
        tokens=3000, hidden=256, heads=8, kv_heads=2, head_dim=64,
        cu=torch.tensor([0, 1100, 3000], dtype=torch.int32),
        attention_config=StreamingAttentionConfig(q_chunk_tokens=768, kv_chunk_tokens=512),
        projection_chunk=512, causal=causal, seed=7,
    )
    _, proj, hidden_cpu, host_out, host_stats = run_pipeline("host", torch.bfloat16, **kwargs)
    _, _, _, hbm_out, hbm_stats = run_pipeline("hbm", torch.bfloat16, **kwargs)
    assert torch.equal(host_out, hbm_out)
    expected, _ = proj.expected(hidden_cpu, [0, 1100, 3000], projection_chunk=512, q_chunk=768,
                                kv_chunk=512, causal=causal, dtype=torch.bfloat16)
    check_projected(hbm_out, expected)
    assert host_stats.attention.h2d_bytes > 0 and hbm_stats.attention.h2d_bytes == 0


@pytest.mark.parametrize("residency", ["host", "hbm"])
def test_projected_runner_reuse_has_bounded_allocator_growth(residency):
    """Reference test_pipeline.py:117-190."""
    announce(f"projected runner reuse {residency}")
    torch.manual_seed(103)
    dtype = torch.bfloat16
    tokens, hidden, heads, head_dim = 257, 64, 4, 16
    hidden_cpu = torch.randn(tokens, hidden, dtype=dtype).pin_memory()
    cu = torch.tensor([0, tokens], dtype=torch.int32)
    proj = Projections(hidden, heads, heads, head_dim, hidden, dtype, 104)
    config = StreamingAttentionConfig(
        backend="triton", q_chunk_tokens=128, kv_chunk_tokens=96, block_m=32, block_n=32, num_output_buffers=2
    )
    plan = build_plan(q_heads=heads, kv_heads=heads, head_dim=head_dim, dtype=dtype, device="cuda",
                      max_q_tokens=tokens, max_kv_tokens=tokens, config=config)
    runner = ProjectedAttentionRunner(
        plan, config, ProjectionPipelineConfig(projection_chunk_tokens=96, qkv_residency=residency)
    )
    out = torch.empty((tokens, hidden), dtype=dtype).pin_memory()
    runner(hidden_cpu, cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector, out=out)
    torch.cuda.synchronize()
    first = out.clone()
    baseline = torch.cuda.memory_allocated()
    for _ in range(10):
        runner(hidden_cpu, cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector, out=out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() <= baseline + 4 * 2**20
    assert torch.equal(out, first)


def test_functional_wrapper_and_projection_errors():
    announce("projected functional wrapper + errors")
    dtype = torch.bfloat16
    tokens, hidden, heads, head_dim = 200, 64, 2, 32
    hidden_cpu = torch.randn(tokens, hidden, generator=torch.Generator().manual_seed(5)).to(dtype).pin_memory()
    proj = Projections(hidden, heads, heads, head_dim, 80, dtype, 6)
    cu = torch.tensor([0, 120, 200], dtype=torch.int32)
    out = streaming_projected_self_attention(
        hidden_cpu, cu, q_heads=heads, kv_heads=heads, head_dim=head_dim,
        project_qkv=proj.project_qkv, output_projector=proj.output_projector, output_features=80,
        pipeline_config=ProjectionPipelineConfig(projection_chunk_tokens=64), causal=True,
    )
    assert out.shape == (tokens, 80) and out.is_pinned()
    expected, _ = proj.expected(hidden_cpu, cu.tolist(), projection_chunk=64, q_chunk=tokens,
                                kv_chunk=tokens, causal=True, dtype=dtype)
    check_projected(out, expected)

    plan = build_plan(q_heads=heads, kv_heads=heads, head_dim=head_dim, dtype=dtype, device="cuda",
                      max_q_tokens=tokens, max_kv_tokens=tokens)
    runner = ProjectedAttentionRunner(plan)

    def bad_projection(hidden_tile, start, stop):
        q, k, v = proj.project_qkv(hidden_tile, start, stop)
        return q[:, :1], k, v

    with pytest.raises(ValueError, match="project_qkv returned q shape"):
        runner(hidden_cpu, cu, project_qkv=bad_projection, output_projector=proj.output_projector,
               output_features=80)
    with pytest.raises(ValueError, match="output_features must be positive"):
        runner(hidden_cpu, cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector)
    with pytest.raises(ValueError, match="pinned hidden_cpu"):
        runner(hidden_cpu.clone(), cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector,
               output_features=80)
    # The runner stays usable after a failed call.
    again = runner(hidden_cpu, cu, project_qkv=proj.project_qkv, output_projector=proj.output_projector,
                   output_features=80, causal=True)
    check_projected(again, expected)
