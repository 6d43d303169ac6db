"""Host-side checks of the projected pipeline (no GPU needed): config
validation as in the reference's tests/test_pipeline.py:16-20, module paths
and the construction errors that fire before any device work."""

from __future__ import annotations

import pytest
import torch

import seqattn
from seqattn import ProjectedAttentionRunner, ProjectionPipelineConfig, StreamingAttentionConfig, build_plan


def test_projection_pipeline_config_validation():
    with pytest.raises(ValueError, match="projection_chunk_tokens"):
        ProjectionPipelineConfig(projection_chunk_tokens=0).validate()
    with pytest.raises(ValueError, match="num_projection_buffers"):
        ProjectionPipelineConfig(num_projection_buffers=4).validate()
    with pytest.raises(ValueError, match="qkv_residency"):
        ProjectionPipelineConfig(qkv_residency="nvme").validate()
    defaults = ProjectionPipelineConfig()
    assert (defaults.projection_chunk_tokens, defaults.num_projection_buffers) == (2048, 2)
    assert defaults.require_pinned_hidden and defaults.pin_qkv and defaults.pin_output
    assert defaults.qkv_residency == "host"
    for buffers in (1, 2, 3):
        ProjectionPipelineConfig(num_projection_buffers=buffers, qkv_residency="hbm").validate()


def test_module_paths_export_one_runner():
    from seqattn.pipeline import ProjectedAttentionRunner as legacy
    from seqattn.projection import ProjectedAttentionRunner as packaged
    from seqattn.projection import streaming_projected_self_attention

    assert legacy is ProjectedAttentionRunner and packaged is ProjectedAttentionRunner
    assert seqattn.streaming_projected_self_attention is streaming_projected_self_attention
    for name in ("ProjectedAttentionRunner", "ProjectionPipelineConfig", "ProjectedAttentionStats",
                 "QKVProjector", "OutputProjector", "streaming_projected_self_attention"):
        assert name in seqattn.__all__


def test_runner_requires_a_gpu_device_and_the_native_backend():
    plan = build_plan(q_heads=4, kv_heads=4, head_dim=16, dtype=torch.bfloat16, device="cpu",
                      max_q_tokens=97, max_kv_tokens=97)
    with pytest.raises(ValueError, match="requires a CUDA device"):
        ProjectedAttentionRunner(plan)
    with pytest.raises(ValueError, match="projection_chunk_tokens"):
        ProjectedAttentionRunner(plan, None, ProjectionPipelineConfig(projection_chunk_tokens=-1))
    with pytest.raises(ValueError, match="unsupported backend"):
        ProjectedAttentionRunner(plan, StreamingAttentionConfig(backend="cuda"))


def test_projected_stats_totals():
    stats = seqattn.ProjectedAttentionStats(projection_hidden_h2d_bytes=10, projection_qkv_d2h_bytes=30)
    stats.attention.h2d_bytes = 5
    stats.attention.d2h_bytes = 7
    totals = stats.as_dict()
    assert totals["total_h2d_bytes"] == 15 and totals["total_d2h_bytes"] == 37
