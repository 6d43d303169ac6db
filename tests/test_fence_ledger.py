"""Ordering of the native transfer pipeline, checked on the CPU.

stream-attn_amd/csrc/sa_pipeline.cpp is compiled with the host compiler
against a recording stand-in of the HIP runtime (tests/native/): every copy,
kernel launch, event record, stream wait and host synchronization lands in a
ledger with the byte ranges it reads and writes, and the ledger checks that
every pair of conflicting accesses is ordered by stream order, event waits
or host synchronization, and that every output copy to the host is complete
when a call returns.  This is the correctness contract of the reference's
event discipline (streaming/executor.py:53-184): no K/V ring slot is refilled
before every launch reading it (both halves of a split chunk) has finished,
no Q block or output slot is overwritten before its readers finish, and no
launch reads a slot before its copy lands.

A mistake planted in the stand-in (one stream wait turned into a no-op) must
be reported, which shows the check can fail.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from seqattn import _native
from seqattn.planner import head_group_unit_sizes

ROOT = Path(__file__).resolve().parents[1]
HEAD_BYTES = 2  # bf16


@pytest.fixture(scope="module")
def ledger(tmp_path_factory):
    compiler = shutil.which("g++")
    if compiler is None:
        pytest.skip("g++ is not available")
    out = tmp_path_factory.mktemp("ledger") / "libfence_ledger.so"
    cmd = [compiler, "-shared", "-fPIC", "-std=c++17", "-O1", f"-I{ROOT / 'tests' / 'native' / 'hip_stub'}",
           f"-I{ROOT / 'include'}", f"-I{ROOT / 'stream-attn_amd' / 'csrc'}",
           str(ROOT / "stream-attn_amd" / "csrc" / "sa_pipeline.cpp"), str(ROOT / "tests" / "native" / "fence_ledger.cpp"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lib = ctypes.CDLL(str(out))
    for name, (restype, argtypes) in _native.SIGNATURES.items():
        if name.startswith("sa_pipeline") or name in ("sa_last_error", "sa_abi_version"):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = restype, argtypes
    lib.ledger_check.restype = ctypes.c_int64
    lib.ledger_check.argtypes = [ctypes.c_char_p, ctypes.c_int64]
    lib.ledger_drop_wait.argtypes = [ctypes.c_long]
    lib.ledger_waits.restype = ctypes.c_long
    lib.ledger_dropped.restype = ctypes.c_long
    lib.ledger_counts.argtypes = [ctypes.POINTER(ctypes.c_int64)]
    lib.ledger_fail_copy.argtypes = [ctypes.c_long]
    lib.ledger_copies.restype = ctypes.c_long
    lib.ledger_unfinished.restype = ctypes.c_int64
    return lib


class Space:
    """Distinct fake address ranges (never dereferenced: the stand-in only records them)."""

    def __init__(self, base: int) -> None:
        self.next = base

    def take(self, nbytes: int) -> int:
        address = self.next
        self.next += (nbytes + (1 << 20)) // (1 << 20) * (1 << 20) + (1 << 20)
        return address


class Pipeline:
    def __init__(self, lib, *, q_chunk, kv_chunk, q_heads, kv_heads, head_dim, num_kv, num_out, out_slots=True):
        dev = Space(0x7000_0000_0000)
        q_row = q_heads * head_dim * HEAD_BYTES
        kv_row = kv_heads * head_dim * HEAD_BYTES
        self.lib = lib
        self.q_buffer = dev.take(q_chunk * q_row)
        k_slots = [dev.take(kv_chunk * kv_row) for _ in range(num_kv)]
        v_slots = [dev.take(kv_chunk * kv_row) for _ in range(num_kv)]
        state_rows = -(-q_chunk // 16) * 16  # the pipeline's state is kept in 16-row groups
        self.m = dev.take(state_rows * q_heads * 4)
        self.l = dev.take(state_rows * q_heads * 4)
        self.acc = dev.take(state_rows * q_heads * head_dim * 4)
        self.out_slots = [dev.take(q_chunk * q_row) for _ in range(num_out)] if out_slots else []
        self.device_space = dev
        self.q_row, self.kv_row, self.q_heads = q_row, kv_row, q_heads
        handle = ctypes.c_void_p()
        ks = (ctypes.c_void_p * 3)(*k_slots)
        vs = (ctypes.c_void_p * 3)(*v_slots)
        outs = (ctypes.c_void_p * 2)(*self.out_slots) if out_slots else None
        status = lib.sa_pipeline_create(ctypes.byref(handle), 0, self.q_buffer, ks, vs, num_kv, self.m, self.l,
                                         self.acc, outs, num_out, q_chunk, kv_chunk, q_heads, kv_heads, head_dim, 0,
                                         None, None)
        assert status == 0, lib.sa_last_error()
        self.handle = handle
        self.compute = 0xC0FFEE  # the caller's compute stream handle

    def destroy(self):
        assert self.lib.sa_pipeline_destroy(self.handle) == 0


def bounds(lengths):
    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return (ctypes.c_int64 * len(out))(*out), out


def check(lib, label):
    msg = ctypes.create_string_buffer(2048)
    violations = lib.ledger_check(msg, len(msg))
    assert violations == 0, f"{label}: {violations} unordered conflicts: {msg.value.decode()}"


def run_tensor_mode(lib, *, num_kv, num_out, causal, q_lengths, k_lengths, q_chunk=1024, kv_chunk=256,
                    q_heads=4, kv_heads=2, head_dim=64, with_lse=True, out_slots=True):
    p = Pipeline(lib, q_chunk=q_chunk, kv_chunk=kv_chunk, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
                 num_kv=num_kv, num_out=num_out, out_slots=out_slots)
    host = Space(0x5000_0000_0000)
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)
    q_host = host.take(q_b[-1] * p.q_row)
    k_host = host.take(k_b[-1] * p.kv_row)
    v_host = host.take(k_b[-1] * p.kv_row)
    out_host = host.take(q_b[-1] * p.q_row)
    lse = p.device_space.take(q_heads * q_b[-1] * 4) if with_lse else None
    stats = _native.PipelineStats()
    status = lib.sa_pipeline_run(p.handle, q_host, k_host, v_host, out_host, lse, q_b[-1] if with_lse else 0,
                                 cu_q, cu_k, len(q_lengths), 0.125, int(causal), p.compute, ctypes.byref(stats))
    assert status == 0, lib.sa_last_error()
    p.destroy()
    return stats


CASES = [
    # (q segment lengths, k segment lengths): several passes per segment, a
    # Q block above 512 rows (split launches), a short last pass, ragged chunks.
    ([3000, 700], [2600, 900]),
    ([1500], [1500]),
    ([200, 0, 3100], [500, 300, 2049]),
]


@pytest.mark.parametrize("num_kv", [1, 2, 3])
@pytest.mark.parametrize("num_out", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
def test_tensor_mode_schedule_is_race_free(ledger, num_kv, num_out, causal):
    for q_lengths, k_lengths in CASES:
        ledger.ledger_reset()
        stats = run_tensor_mode(ledger, num_kv=num_kv, num_out=num_out, causal=causal, q_lengths=q_lengths,
                                k_lengths=k_lengths)
        counts = (ctypes.c_int64 * 4)()
        ledger.ledger_counts(counts)
        assert counts[0] > 0 and counts[1] > 0 and counts[2] > 0
        assert stats.d2h_bytes == sum(q_lengths) * 4 * 64 * HEAD_BYTES
        check(ledger, f"num_kv={num_kv} num_out={num_out} causal={causal} q={q_lengths} k={k_lengths}")


@pytest.mark.parametrize("num_kv", [1, 2, 3])
@pytest.mark.parametrize("causal", [False, True])
def test_host_aliased_schedule_is_race_free(ledger, num_kv, causal):
    # output_mode="host_aliased": no output slot; each block is finalized
    # into the Q buffer and copied out from it, and the next block's first
    # K/V chunk is copied before its Q block.
    for q_lengths, k_lengths in CASES:
        ledger.ledger_reset()
        stats = run_tensor_mode(ledger, num_kv=num_kv, num_out=1, causal=causal, q_lengths=q_lengths,
                                k_lengths=k_lengths, out_slots=False)
        assert stats.d2h_bytes == sum(q_lengths) * 4 * 64 * HEAD_BYTES
        check(ledger, f"host_aliased num_kv={num_kv} causal={causal} q={q_lengths} k={k_lengths}")


@pytest.mark.parametrize("causal", [False, True])
def test_host_aliased_pieces_at_head_dim_128_are_race_free(ledger, causal):
    # The GPU test's shapes: 384-row workgroup tiles, blocks of 3-4 tiles
    # (3-4 pieces), a segment with fewer keys than queries and one with fewer
    # keys than a chunk (single-chunk passes).
    ledger.ledger_reset()
    stats = run_tensor_mode(ledger, num_kv=2, num_out=1, causal=causal, q_lengths=[2000, 1300, 500],
                            k_lengths=[1800, 1200, 200], q_chunk=1536, kv_chunk=256, q_heads=8, kv_heads=2,
                            head_dim=128, out_slots=False)
    assert stats.d2h_bytes == 3800 * 8 * 128 * HEAD_BYTES
    check(ledger, f"host_aliased d128 causal={causal}")


def test_step_api_schedules_are_race_free(ledger):
    # The per-Q-block steps the Python executor drives for device consumers
    # and device outputs (seqattn/streaming/executor.py): output slots with
    # D2H, the output finalized into the Q buffer and released by the D2H,
    # and the output finalized straight into caller device memory.
    for num_kv, num_out in ((1, 1), (2, 2), (3, 1)):
        ledger.ledger_reset()
        p = Pipeline(ledger, q_chunk=1024, kv_chunk=256, q_heads=4, kv_heads=2, head_dim=64, num_kv=num_kv,
                     num_out=num_out)
        host = Space(0x5000_0000_0000)
        n_q, n_k = 2900, 2300
        q_host, k_host, v_host = host.take(n_q * p.q_row), host.take(n_k * p.kv_row), host.take(n_k * p.kv_row)
        out_host = host.take(n_q * p.q_row)
        out_dev = p.device_space.take(n_q * p.q_row)
        for mode in ("slots", "q_reuse", "device_out"):
            for index, start in enumerate(range(0, n_q, 1024)):
                rows = min(1024, n_q - start)
                assert ledger.sa_pipeline_load_q(p.handle, q_host + start * p.q_row, rows, p.compute, None) == 0
                assert ledger.sa_pipeline_stream_kv(p.handle, k_host, v_host, n_k, rows, start, n_k - n_q, 0.125, 0,
                                                    p.compute, None) == 0
                slot = index % num_out
                if mode == "slots":
                    assert ledger.sa_pipeline_finalize(p.handle, slot, rows, None, 0, start, p.compute) == 0
                    assert ledger.sa_pipeline_d2h(p.handle, out_host + start * p.q_row, p.out_slots[slot],
                                                  rows * p.q_row, slot, 0, p.compute, None) == 0
                elif mode == "q_reuse":
                    assert ledger.sa_pipeline_finalize(p.handle, -1, rows, None, 0, start, p.compute) == 0
                    assert ledger.sa_pipeline_d2h(p.handle, out_host + start * p.q_row, p.q_buffer, rows * p.q_row,
                                                  slot, 1, p.compute, None) == 0
                else:
                    assert ledger.sa_pipeline_finalize_into(p.handle, out_dev + start * p.q_row, 4 * 64, 64, rows,
                                                            None, 0, start, p.compute) == 0
            assert ledger.sa_pipeline_synchronize(p.handle) == 0
        p.destroy()
        check(ledger, f"step API num_kv={num_kv} num_out={num_out}")


def test_resident_schedule_with_transposed_v_scratch_is_race_free(ledger):
    ledger.ledger_reset()
    p = Pipeline(ledger, q_chunk=1024, kv_chunk=256, q_heads=4, kv_heads=4, head_dim=128, num_kv=2, num_out=1)
    dev = p.device_space
    cu_q, q_b = bounds([700, 1900])
    cu_k, k_b = bounds([900, 1300])
    row = 4 * 128 * HEAD_BYTES
    q, k, v, out = dev.take(q_b[-1] * row), dev.take(k_b[-1] * row), dev.take(k_b[-1] * row), dev.take(q_b[-1] * row)
    scratch_bytes = 4 * 128 * 1344 * HEAD_BYTES
    assert ledger.sa_pipeline_attach_resident_scratch(p.handle, dev.take(scratch_bytes), scratch_bytes) == 0
    lse = dev.take(4 * q_b[-1] * 4)
    status = ledger.sa_pipeline_run_resident(p.handle, q, k, v, out, lse, 512, 128, 512, 128, 512, 128, 512, 128,
                                             q_b[-1], cu_q, cu_k, 2, 0.09, 1, p.compute, None)
    assert status == 0, ledger.sa_last_error()
    p.destroy()
    check(ledger, "resident")


def test_a_dropped_wait_is_reported(ledger):
    # Every stream wait of one run is dropped in turn.  The waits that keep a
    # K/V slot, the Q block / output slot pair or the D2H ordered are
    # necessary, so most drops must be reported (63 of 69 here); the rest are
    # waits another ordering already implies.
    def run():
        run_tensor_mode(ledger, num_kv=2, num_out=1, causal=False, q_lengths=[3000], k_lengths=[1100])

    ledger.ledger_reset()
    run()
    check(ledger, "baseline")
    waits = ledger.ledger_waits()
    assert waits > 10
    caught = 0
    for n in range(waits):
        ledger.ledger_reset()
        ledger.ledger_drop_wait(n)
        run()
        assert ledger.ledger_dropped() == 1
        caught += ledger.ledger_check(None, 0) > 0
    print(f"dropped-wait runs reported: {caught} of {waits}")
    assert caught >= waits * 3 // 4


def test_a_dropped_wait_is_reported_in_host_aliased_runs(ledger):
    # The same mutation check for the host_aliased schedule, whose Q block
    # doubles as the output buffer: the waits that keep the next block's Q
    # copy behind the previous block's output copy, and the prefetched first
    # chunk behind the slot's last readers, must be among those reported.
    def run():
        run_tensor_mode(ledger, num_kv=2, num_out=1, causal=False, q_lengths=[3000], k_lengths=[1100],
                        out_slots=False)

    ledger.ledger_reset()
    run()
    check(ledger, "baseline")
    waits = ledger.ledger_waits()
    assert waits > 10
    caught = 0
    for n in range(waits):
        ledger.ledger_reset()
        ledger.ledger_drop_wait(n)
        run()
        assert ledger.ledger_dropped() == 1
        caught += ledger.ledger_check(None, 0) > 0
    print(f"host_aliased dropped-wait runs reported: {caught} of {waits}")
    assert caught >= waits * 3 // 4


def run_head_groups(lib, *, num_sets, causal, q_lengths, k_lengths, group_kv, q_heads=4, kv_heads=2, head_dim=64,
                    kv_chunk=256, with_vt=False, with_lse=True):
    """One sa_pipeline_run on a head-group pipeline (every token of a group
    of K/V heads per unit, buffer sets used in turn)."""
    dev = Space(0x7000_0000_0000)
    host = Space(0x5000_0000_0000)
    group = q_heads // kv_heads
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)
    tq, tk = q_b[-1], k_b[-1]
    qo = [dev.take(tq * group_kv * group * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    ks = [dev.take(tk * group_kv * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    vs = [dev.take(tk * group_kv * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    vt_bytes = group_kv * 128 * (-(-max(k_lengths) // 64) * 64) * HEAD_BYTES if with_vt else 0
    vts = (ctypes.c_void_p * 2)(*[dev.take(vt_bytes) for _ in range(num_sets)]) if with_vt else None
    handle = ctypes.c_void_p()
    status = lib.sa_pipeline_create_head_groups(
        ctypes.byref(handle), 0, (ctypes.c_void_p * 2)(*qo), (ctypes.c_void_p * 2)(*ks), (ctypes.c_void_p * 2)(*vs),
        vts, vt_bytes, num_sets, tq, tk, group_kv, kv_chunk, q_heads, kv_heads, head_dim, 0, None, None)
    assert status == 0, lib.sa_last_error()
    q_row, kv_row = q_heads * head_dim * HEAD_BYTES, kv_heads * head_dim * HEAD_BYTES
    q_host, k_host, v_host = host.take(tq * q_row), host.take(tk * kv_row), host.take(tk * kv_row)
    out_host = host.take(tq * q_row)
    lse = dev.take(q_heads * tq * 4) if with_lse else None
    stats = _native.PipelineStats()
    status = lib.sa_pipeline_run(handle, q_host, k_host, v_host, out_host, lse, tq if with_lse else 0, cu_q, cu_k,
                                 len(q_lengths), 0.125, int(causal), 0xC0FFEE, ctypes.byref(stats))
    assert status == 0, lib.sa_last_error()
    assert lib.sa_pipeline_destroy(handle) == 0
    return stats


HEAD_GROUP_CASES = [
    # (q_heads, kv_heads, K/V heads per unit): MHA one head per unit, GQA
    # with a short last group, all heads in one unit.
    (4, 4, 1),
    (8, 4, 3),
    (6, 2, 2),
]


@pytest.mark.parametrize("num_sets", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads", HEAD_GROUP_CASES)
def test_head_group_schedule_is_race_free(ledger, num_sets, causal, heads):
    q_heads, kv_heads, group_kv = heads
    for q_lengths, k_lengths in CASES:
        ledger.ledger_reset()
        stats = run_head_groups(ledger, num_sets=num_sets, causal=causal, q_lengths=q_lengths, k_lengths=k_lengths,
                                group_kv=group_kv, q_heads=q_heads, kv_heads=kv_heads)
        units = len(head_group_unit_sizes(kv_heads, group_kv, num_sets))
        row = q_heads * 64 * HEAD_BYTES
        # Every byte of Q, K and V crosses the link once; the output once.
        assert stats.h2d_bytes == sum(q_lengths) * row + 2 * sum(k_lengths) * kv_heads * 64 * HEAD_BYTES
        assert stats.d2h_bytes == sum(q_lengths) * row
        assert stats.q_chunks == units
        counts = (ctypes.c_int64 * 4)()
        ledger.ledger_counts(counts)
        assert counts[0] == 3 * units and counts[1] == units
        assert counts[2] == units * sum(1 for n in q_lengths if n > 0)
        check(ledger, f"head groups sets={num_sets} causal={causal} heads={heads} q={q_lengths} k={k_lengths}")


@pytest.mark.parametrize("num_sets", [1, 2])
def test_head_group_schedule_with_transposed_v_is_race_free(ledger, num_sets):
    ledger.ledger_reset()
    run_head_groups(ledger, num_sets=num_sets, causal=True, q_lengths=[700, 0, 1900], k_lengths=[900, 40, 1300],
                    group_kv=1, q_heads=8, kv_heads=4, head_dim=128, with_vt=True)
    counts = (ctypes.c_int64 * 4)()
    ledger.ledger_counts(counts)
    assert counts[2] == 4 * 2 * 2  # per unit and non-empty segment: a transpose and an update launch
    check(ledger, f"head groups with transposed V, sets={num_sets}")


def test_a_dropped_wait_is_reported_in_head_group_runs(ledger):
    # The waits that hold a set's next copies behind its previous output copy,
    # a unit's launch behind its copies and the output copy behind the launch
    # are all necessary; only the fork and join of the second stream can be
    # implied by other orderings.
    def run():
        run_head_groups(ledger, num_sets=2, causal=False, q_lengths=[1500, 900], k_lengths=[1200, 900], group_kv=1,
                        q_heads=4, kv_heads=4)

    ledger.ledger_reset()
    run()
    check(ledger, "baseline")
    waits = ledger.ledger_waits()
    assert waits > 10
    caught = 0
    for n in range(waits):
        ledger.ledger_reset()
        ledger.ledger_drop_wait(n)
        run()
        assert ledger.ledger_dropped() == 1
        caught += ledger.ledger_check(None, 0) > 0
    print(f"head-group dropped-wait runs reported: {caught} of {waits}")
    assert caught >= waits - 2


def test_step_api_is_refused_on_head_group_pipelines(ledger):
    dev = Space(0x7000_0000_0000)
    bufs = (ctypes.c_void_p * 2)(dev.take(1 << 20), dev.take(1 << 20))
    handle = ctypes.c_void_p()
    assert ledger.sa_pipeline_create_head_groups(ctypes.byref(handle), 0, bufs, bufs, bufs, None, 0, 1, 1024, 1024, 1,
                                                 256, 4, 4, 64, 0, None, None) == 0
    assert ledger.sa_pipeline_load_q(handle, 0x5000_0000_0000, 16, 0xC0FFEE, None) == -4
    assert b"head-group" in ledger.sa_last_error()
    assert ledger.sa_pipeline_finalize(handle, 0, 16, None, 0, 0, 0xC0FFEE) == -4
    assert ledger.sa_pipeline_release_q(handle, 0xC0FFEE) == -4
    assert ledger.sa_pipeline_destroy(handle) == 0


def test_head_group_schedule_with_host_staging_is_race_free(ledger):
    # A pageable output goes through page-locked staging in row chunks: on
    # the D2H stream a chunk's copy, then a host function scattering it into
    # the host rows (the staging and the output are real host memory here:
    # the scatter runs).  The ledger checks the device-side order: each set's
    # next copies after its output left, each staging copy after the unit's
    # launches and after the previous chunk's scatter.
    import numpy as np

    q_heads, kv_heads, head_dim = 4, 4, 64
    q_lengths, k_lengths = [1500, 900], [1200, 900]
    tq = sum(q_lengths)
    row = q_heads * head_dim * HEAD_BYTES
    staging = np.zeros(8192, dtype=np.uint8)  # 64 output rows of one head
    out = np.zeros(tq * row, dtype=np.uint8)
    dev = Space(0x7000_0000_0000)
    host = Space(0x5000_0000_0000)
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)
    for num_sets in (1, 2):
        ledger.ledger_reset()
        qo = [dev.take(tq * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        ks = [dev.take(k_b[-1] * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        vs = [dev.take(k_b[-1] * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        handle = ctypes.c_void_p()
        assert ledger.sa_pipeline_create_head_groups(
            ctypes.byref(handle), 0, (ctypes.c_void_p * 2)(*qo), (ctypes.c_void_p * 2)(*ks),
            (ctypes.c_void_p * 2)(*vs), None, 0, num_sets, tq, k_b[-1], 1, 256, q_heads, kv_heads, head_dim, 0, None,
            None) == 0
        assert ledger.sa_pipeline_attach_host_staging(handle, staging.ctypes.data, staging.nbytes) == 0
        q_host, k_host, v_host = host.take(tq * row), host.take(k_b[-1] * row), host.take(k_b[-1] * row)
        stats = _native.PipelineStats()
        status = ledger.sa_pipeline_run(handle, q_host, k_host, v_host, out.ctypes.data, None, 0, cu_q, cu_k, 2,
                                        0.125, 0, 0xC0FFEE, ctypes.byref(stats))
        assert status == 0, ledger.sa_last_error()
        assert stats.d2h_bytes == tq * row
        counts = (ctypes.c_int64 * 4)()
        ledger.ledger_counts(counts)
        chunks = 4 * -(-tq // 64)  # per unit one staging copy and one scatter per 64-row chunk
        assert counts[1] == chunks
        assert counts[2] == 4 * 2 + chunks  # update launches per unit and segment, and the scatters
        check(ledger, f"head groups with host staging, sets={num_sets}")
        assert ledger.sa_pipeline_destroy(handle) == 0
    # Staging smaller than one output row is refused before anything runs.
    handle = ctypes.c_void_p()
    bufs = (ctypes.c_void_p * 2)(dev.take(1 << 20), dev.take(1 << 20))
    assert ledger.sa_pipeline_create_head_groups(ctypes.byref(handle), 0, bufs, bufs, bufs, None, 0, 1, 1024, 1024, 4,
                                                 256, 64, 4, 256, 0, None, None) == 0
    assert ledger.sa_pipeline_attach_host_staging(handle, staging.ctypes.data, staging.nbytes) == 0
    ledger.ledger_reset()
    cu = (ctypes.c_int64 * 2)(0, 512)
    assert ledger.sa_pipeline_run(handle, 0x5000_0000_0000, 0x5100_0000_0000, 0x5200_0000_0000, out.ctypes.data, None,
                                  0, cu, cu, 1, 0.1, 0, 0xC0FFEE, None) == -1
    assert b"host staging" in ledger.sa_last_error()
    counts = (ctypes.c_int64 * 4)()
    ledger.ledger_counts(counts)
    assert list(counts) == [0, 0, 0, 0]
    assert ledger.sa_pipeline_destroy(handle) == 0


@pytest.mark.parametrize("num_sets", [1, 2])
def test_head_group_schedule_into_device_output_is_race_free(ledger, num_sets):
    # The unit launches write the caller's device rows of their heads; no
    # output copy.  A set's next copies wait for its launches, and the
    # call returns after the last input copy landed.
    q_heads, kv_heads, head_dim = 6, 3, 64
    q_lengths, k_lengths = [1500, 0, 900], [1200, 40, 900]
    dev = Space(0x7000_0000_0000)
    host = Space(0x5000_0000_0000)
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)
    tq, tk = q_b[-1], k_b[-1]
    qo = [dev.take(tq * 2 * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    ks = [dev.take(tk * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    vs = [dev.take(tk * head_dim * HEAD_BYTES) for _ in range(num_sets)]
    ledger.ledger_reset()
    handle = ctypes.c_void_p()
    assert ledger.sa_pipeline_create_head_groups(
        ctypes.byref(handle), 0, (ctypes.c_void_p * 2)(*qo), (ctypes.c_void_p * 2)(*ks), (ctypes.c_void_p * 2)(*vs),
        None, 0, num_sets, tq, tk, 1, 256, q_heads, kv_heads, head_dim, 0, None, None) == 0
    row = q_heads * head_dim * HEAD_BYTES
    q_host, k_host = host.take(tq * row), host.take(tk * kv_heads * head_dim * HEAD_BYTES)
    v_host = host.take(tk * kv_heads * head_dim * HEAD_BYTES)
    out = dev.take(tq * row)
    lse = dev.take(q_heads * tq * 4)
    stats = _native.PipelineStats()
    status = ledger.sa_pipeline_run_device_output(handle, q_host, k_host, v_host, out, q_heads * head_dim, head_dim,
                                                  lse, tq, cu_q, cu_k, 3, 0.125, 1, 0xC0FFEE, ctypes.byref(stats))
    assert status == 0, ledger.sa_last_error()
    assert stats.d2h_bytes == 0
    counts = (ctypes.c_int64 * 4)()
    ledger.ledger_counts(counts)
    assert counts[1] == 0 and counts[2] == 3 * 2
    check(ledger, f"head groups into device output, sets={num_sets}")
    # misaligned output strides are refused before anything is enqueued
    ledger.ledger_reset()
    assert ledger.sa_pipeline_run_device_output(handle, q_host, k_host, v_host, out, q_heads * head_dim + 4,
                                                head_dim, None, 0, cu_q, cu_k, 3, 0.125, 0, 0xC0FFEE, None) == -1
    ledger.ledger_counts(counts)
    assert list(counts) == [0, 0, 0, 0]
    assert ledger.sa_pipeline_destroy(handle) == 0


def _failing_runs(ledger, run, label):
    """Make each copy of a run fail in turn: the call reports the error, and
    no copy it enqueued (nor a host function) is still running when it
    returns, so the caller may release its buffers."""
    ledger.ledger_reset()
    status, unfinished = run()
    assert status == 0 and unfinished == 0, label
    copies = ledger.ledger_copies()
    assert copies > 3
    for n in range(copies):
        ledger.ledger_reset()
        ledger.ledger_fail_copy(n)
        status, unfinished = run()
        assert status != 0, f"{label}: copy {n} failed, the run reported success"
        assert unfinished == 0, f"{label}: copy {n} failed, {unfinished} copies in flight at the return"


@pytest.mark.parametrize("num_out,out_slots", [(1, True), (2, True), (0, False)])
def test_a_failed_tensor_mode_run_returns_with_its_copies_drained(ledger, num_out, out_slots):
    host = Space(0x5000_0000_0000)
    q_lengths, k_lengths = [3000, 700], [2600, 900]
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)

    def run():
        p = Pipeline(ledger, q_chunk=1024, kv_chunk=256, q_heads=4, kv_heads=2, head_dim=64, num_kv=2,
                     num_out=max(num_out, 1), out_slots=out_slots)
        q_host, k_host = host.take(q_b[-1] * p.q_row), host.take(k_b[-1] * p.kv_row)
        v_host, out_host = host.take(k_b[-1] * p.kv_row), host.take(q_b[-1] * p.q_row)
        status = ledger.sa_pipeline_run(p.handle, q_host, k_host, v_host, out_host, None, 0, cu_q, cu_k, 2, 0.125, 0,
                                        p.compute, None)
        unfinished = ledger.ledger_unfinished()
        p.destroy()
        return status, unfinished

    _failing_runs(ledger, run, f"tensor mode, {num_out} output slots")


@pytest.mark.parametrize("num_sets", [1, 2])
@pytest.mark.parametrize("device_output", [False, True])
def test_a_failed_head_group_run_returns_with_its_copies_drained(ledger, num_sets, device_output):
    q_heads, kv_heads, head_dim = 4, 4, 64
    q_lengths, k_lengths = [1500, 900], [1200, 900]
    dev = Space(0x7000_0000_0000)
    host = Space(0x5000_0000_0000)
    cu_q, q_b = bounds(q_lengths)
    cu_k, k_b = bounds(k_lengths)
    tq, tk = q_b[-1], k_b[-1]
    row = q_heads * head_dim * HEAD_BYTES

    def run():
        qo = [dev.take(tq * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        ks = [dev.take(tk * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        vs = [dev.take(tk * head_dim * HEAD_BYTES) for _ in range(num_sets)]
        handle = ctypes.c_void_p()
        assert ledger.sa_pipeline_create_head_groups(
            ctypes.byref(handle), 0, (ctypes.c_void_p * 2)(*qo), (ctypes.c_void_p * 2)(*ks),
            (ctypes.c_void_p * 2)(*vs), None, 0, num_sets, tq, tk, 1, 256, q_heads, kv_heads, head_dim, 0, None,
            None) == 0
        q_host, k_host, v_host = host.take(tq * row), host.take(tk * row), host.take(tk * row)
        if device_output:
            status = ledger.sa_pipeline_run_device_output(handle, q_host, k_host, v_host, dev.take(tq * row),
                                                          q_heads * head_dim, head_dim, None, 0, cu_q, cu_k, 2,
                                                          0.125, 0, 0xC0FFEE, None)
        else:
            status = ledger.sa_pipeline_run(handle, q_host, k_host, v_host, host.take(tq * row), None, 0, cu_q,
                                            cu_k, 2, 0.125, 0, 0xC0FFEE, None)
        unfinished = ledger.ledger_unfinished()
        assert ledger.sa_pipeline_destroy(handle) == 0
        return status, unfinished

    _failing_runs(ledger, run, f"head groups, sets={num_sets}, device output={device_output}")

