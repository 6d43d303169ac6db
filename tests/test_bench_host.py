"""Host-side pieces of bench.py: the one-GPU guard, the traffic-summary reader,
the CPU-share rule, the seeded inputs and the sampled-row parity check.

No GPU: the parity check runs on CPU tensors standing in for the device
result, with the float64 dense oracle as the expected values.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import bench
from oracle.seqattn_oracle import dense_attention_f64, seeded_normal_chunks

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=60)
    assert done.returncode == 2
    assert "one GPU" in done.stderr
    assert done.stdout == ""


def test_read_traffic_takes_the_first_bytes_line(tmp_path):
    f = tmp_path / "t.txt"
    f.write_text("command: rocprofv3 --pmc FETCH_SIZE\nFETCH_SIZE: 12 KiB\nbytes_per_span: 1.5e9\n"
                 "bytes_per_launch: 7\n")
    assert bench.read_traffic(f) == 1.5e9
    f.write_text("note\n  bytes_per_launch:  42\n")
    assert bench.read_traffic(f) == 42.0
    f.write_text("FETCH_SIZE: 12\n")
    assert bench.read_traffic(f) is None
    assert bench.read_traffic(tmp_path / "missing.txt") is None


def test_committed_traffic_summary_parses():
    value = bench.read_traffic(ROOT / "profiles" / "update_kernel_pinned_524k_56h_2gib_traffic.txt")
    assert value is not None and value > 0


def test_cpu_share_is_capped_by_omp_num_threads(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    share, info = bench.cpu_share()
    assert share == 1 and info["omp_num_threads"] == 1
    monkeypatch.delenv("OMP_NUM_THREADS")
    share, info = bench.cpu_share()
    assert 1 <= share <= info["affinity_cpus"]
    assert info["omp_num_threads"] is None


def test_make_inputs_follow_the_seeded_chunk_scheme():
    # 9,000 tokens: two full 4,096-token chunks and a ragged one.
    q, k, v = bench.make_inputs(9000, 2, 8, seed=7, workers=4, pinned=False)
    for t, x in enumerate((q, k, v)):
        ref = seeded_normal_chunks(9000, 2, 8, seed=7, tensor_index=t)
        assert torch.equal(x, ref)
    assert not torch.equal(q, k)
    # chunk 1 of tensor 0 restarts from its own generator
    g = torch.Generator(device="cpu").manual_seed(7 + 0 * 1_000_003 + 1)
    first = torch.empty((4096, 2, 8), dtype=torch.bfloat16).normal_(generator=g)
    assert torch.equal(q[4096:8192], first)


def _exact_result(n=300, h=3, d=16, seed=5):
    """Inputs, a bf16 'device' output equal to the float64 oracle rounded, and its LSE."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn((n, h, d), generator=g).to(torch.bfloat16) for _ in range(3))
    o64, lse64 = dense_attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), [0, n], [0, n])
    out = torch.from_numpy(o64.astype(np.float32)).to(torch.bfloat16)
    lse = torch.from_numpy(lse64.astype(np.float32))
    return q, k, v, out, lse


def test_sampled_parity_accepts_the_exact_result_and_times_the_cpu_baseline():
    q, k, v, out, lse = _exact_result()
    rows = np.array([0, 75, 150, 225, 299, 17, 40])
    parity, (seconds, timed, agree, oracle_seconds) = bench.sampled_parity(q, k, v, out, lse, rows, kv_chunk=64,
                                                                           workers=2)
    assert parity["ok"] and parity["rows"] == rows.size
    assert parity["max_abs_o"] < 1e-2 and parity["max_abs_lse"] < 1e-4
    assert seconds > 0 and oracle_seconds > 0 and timed == rows.size
    # The timed torch restatement computes what the oracle computes.
    assert agree["max_abs_o"] < 1e-5 and agree["max_abs_lse"] < 1e-5
    entry = bench.cpu_baseline_entry(4 * 3 * 16 * 300, timed, seconds, 2, "sample", agree, rows.size, oracle_seconds)
    assert entry["kind"] == "port" and entry["cores"] == 2 and entry["value"] > 0
    assert entry["vs_numpy_oracle"] == agree and entry["numpy_oracle_tflops"] > 0


def test_cpu_baseline_sample_is_bounded(monkeypatch):
    # The timed rows are cut to CPU_SAMPLE_FLOP of work; the agreement is
    # taken on those rows.
    q, k, v, out, lse = _exact_result()
    rows = np.arange(0, 300, 3)
    ref_o, ref_l, _ = bench.oracle_sample(q, k, v, rows, kv_chunk=64, workers=1)
    monkeypatch.setattr(bench, "CPU_SAMPLE_FLOP", 4 * 3 * 16 * 300 * 10)
    seconds, timed, agree = bench.torch_cpu_sample(q[torch.from_numpy(rows)], k, v, 64, 1, ref_o, ref_l)
    assert timed == 10 and seconds > 0
    assert agree["max_abs_o"] < 1e-5 and agree["max_abs_lse"] < 1e-5


@pytest.mark.parametrize("mistake", ["o_element", "lse_row", "row_swap", "head_swap"])
def test_compare_sample_rejects_a_planted_mistake(mistake):
    q, k, v, out, lse = _exact_result()
    rows = np.array([3, 50, 120, 299])
    ref_o, ref_l, _ = bench.oracle_sample(q, k, v, rows, kv_chunk=64, workers=1)
    assert bench.compare_sample(out, lse, rows, ref_o, ref_l)["ok"]
    ref_o, ref_l = ref_o.copy(), ref_l.copy()
    if mistake == "o_element":
        ref_o[2, 1, 5] += 0.05
    elif mistake == "lse_row":
        ref_l[0, 1] += 2e-3
    elif mistake == "row_swap":
        ref_o[[0, 1]] = ref_o[[1, 0]]
    else:
        ref_o[:, [0, 2]] = ref_o[:, [2, 0]]
    assert not bench.compare_sample(out, lse, rows, ref_o, ref_l)["ok"]


def test_compare_sample_without_lse_checks_o_only():
    q, k, v, out, _ = _exact_result()
    rows = np.array([1, 2, 3])
    ref_o, ref_l, _ = bench.oracle_sample(q, k, v, rows, kv_chunk=128, workers=1)
    parity = bench.compare_sample(out, None, rows, ref_o, ref_l + 1.0)
    assert parity["ok"] and "max_abs_lse" not in parity
