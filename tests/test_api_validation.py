"""Host-side validation and configuration behaviour (no GPU needed)."""

import pytest
import torch

from seqattn import PagedAttentionConfig, StreamingAttentionConfig, streaming_attn_func
from seqattn.validation import validate_host_qkv


def test_dense_api_rejects_dropout():
    q = torch.randn(1, 2, 1, 8)
    with pytest.raises(ValueError, match="dropout_p=0"):
        streaming_attn_func(q, q, q, dropout_p=0.1, device="cpu")


def test_validation_messages_match_reference():
    q = torch.randn(2, 1, 8)
    k = torch.empty(0, 1, 8)
    with pytest.raises(ValueError, match="queries but no keys"):
        validate_host_qkv(q, k, k, torch.tensor([0, 2]), torch.tensor([0, 0]))
    with pytest.raises(ValueError, match="packed"):
        validate_host_qkv(q[0], k, k, torch.tensor([0, 2]), torch.tensor([0, 0]))
    with pytest.raises(ValueError, match="divisible"):
        validate_host_qkv(torch.randn(2, 3, 8), torch.randn(2, 2, 8), torch.randn(2, 2, 8),
                          torch.tensor([0, 2]), torch.tensor([0, 2]))
    with pytest.raises(ValueError, match="span"):
        validate_host_qkv(q, q, q, torch.tensor([0, 1]), torch.tensor([0, 2]))
    with pytest.raises(ValueError, match="non-decreasing"):
        validate_host_qkv(q, q, q, torch.tensor([0, 3, 2]), torch.tensor([0, 1, 2]))
    bounds = validate_host_qkv(q, q, q, torch.tensor([0, 1, 2]), torch.tensor([0, 0, 2]).clone().index_fill_(0, torch.tensor([1]), 1))
    assert bounds == ([0, 1, 2], [0, 1, 2])


def test_config_validation():
    StreamingAttentionConfig(backend="hip", output_mode="host_aliased").validate()
    for bad in (dict(num_kv_buffers=4), dict(output_mode="x"), dict(block_m=48), dict(backend="cuda")):
        with pytest.raises(ValueError):
            StreamingAttentionConfig(**bad).validate()
    PagedAttentionConfig().validate()
    with pytest.raises(ValueError, match="room for the DRAM cache"):
        PagedAttentionConfig(host_memory_budget_bytes=1 * 2**30).validate()


def test_api_runner_cache_drops_a_runner_whose_call_raised_and_keeps_no_resident_scratch(monkeypatch):
    # The FlashAttention-style wrappers keep the last runner; a stand-in
    # runner (no GPU needed) records what the cache does with it.
    import seqattn.api as api

    events = []

    class FakeRunner:
        def __init__(self, plan, config):
            self.id = len([e for e in events if e[0] == "new"])
            events.append(("new", self.id))

        def close(self):
            events.append(("close", self.id))

        def release_resident_scratch(self):
            events.append(("release", self.id))

    monkeypatch.setattr(api, "StreamingAttentionRunner", FakeRunner)
    api.clear_runner_cache()
    key = ("plan", "config")
    assert api._run_cached(*key, lambda r: "ok") == "ok"
    assert api._run_cached(*key, lambda r: "again") == "again"
    assert events == [("new", 0), ("release", 0), ("release", 0)]

    def boom(runner):
        raise RuntimeError("kernel launch failed")

    with pytest.raises(RuntimeError, match="kernel launch failed"):
        api._run_cached(*key, boom)
    assert events[-1] == ("close", 0) and api._cached is None
    assert api._run_cached(*key, lambda r: r.id) == 1  # a fresh runner
    api.clear_runner_cache()
    assert events[-1] == ("close", 1) and api._cached is None
