"""Pins of the CPU oracle (oracle/seqattn_oracle.py) before it is trusted.

Each check is independent of the oracle's own formula: a float64 closed form,
explicit per-row loops, the reference tests' known answers, chunk-size
invariance and the base-2 / natural-log LSE identity.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import (
    brute_force_row,
    chunked_attention,
    dense_attention_f64,
    seeded_normal_chunks,
)


def bounds(lengths):
    return np.array([0, *itertools.accumulate(lengths)], dtype=np.int64)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(4, 4), (8, 2)])
@pytest.mark.parametrize("q_chunk,kv_chunk", [(3, 2), (8, 5)])
def test_oracle_matches_dense_closed_form(causal, q_heads, kv_heads, q_chunk, kv_chunk):
    # Shapes and tolerance of the reference's tests/test_reference.py:41-64.
    rng = np.random.default_rng(7)
    cu_q, cu_k = bounds([7, 0, 10]), bounds([9, 0, 12])
    q = rng.standard_normal((17, q_heads, 32)).astype(np.float32)
    k = rng.standard_normal((21, kv_heads, 32)).astype(np.float32)
    v = rng.standard_normal((21, kv_heads, 32)).astype(np.float32)
    out, lse = chunked_attention(q, k, v, cu_q, cu_k, q_chunk_tokens=q_chunk, kv_chunk_tokens=kv_chunk,
                                 softmax_scale=0.19, causal=causal)
    ref_o, ref_lse = dense_attention_f64(q, k, v, cu_q, cu_k, softmax_scale=0.19, causal=causal)
    np.testing.assert_allclose(out, ref_o, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(lse, ref_lse, atol=2e-5, rtol=2e-5)


def test_oracle_matches_brute_force_loops():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((6, 2, 8)).astype(np.float32)
    k = rng.standard_normal((9, 1, 8)).astype(np.float32)
    v = rng.standard_normal((9, 1, 8)).astype(np.float32)
    cu_q, cu_k = bounds([6]), bounds([9])
    for causal in (False, True):
        out, lse = chunked_attention(q, k, v, cu_q, cu_k, q_chunk_tokens=4, kv_chunk_tokens=4,
                                     softmax_scale=0.5, causal=causal)
        for t in range(6):
            for h in range(2):
                visible = t + (9 - 6) + 1 if causal else None
                o, ls = brute_force_row(q[t, h].astype(np.float64), k[:, 0].astype(np.float64),
                                        v[:, 0].astype(np.float64), scale=0.5, visible_keys=visible)
                np.testing.assert_allclose(out[t, h], o, atol=1e-5)
                assert abs(lse[h, t] - ls) < 1e-5


def test_oracle_segments_are_isolated():
    # Known answer of the reference's tests/test_reference.py:67-82.
    q = np.ones((4, 1, 8), dtype=np.float32)
    k = np.ones_like(q)
    v = np.concatenate([np.zeros((2, 1, 8)), np.full((2, 1, 8), 10.0)]).astype(np.float32)
    cu = np.array([0, 2, 4])
    out, lse = chunked_attention(q, k, v, cu, cu, q_chunk_tokens=1, kv_chunk_tokens=1)
    np.testing.assert_array_equal(out[:2], 0.0)
    np.testing.assert_allclose(out[2:], 10.0)
    # two equal logits of 8 * 8**-0.5 each
    np.testing.assert_allclose(lse, math.sqrt(8) + math.log(2), rtol=1e-6)


def test_oracle_rejects_query_sequence_without_keys():
    q = np.zeros((2, 1, 8), dtype=np.float32)
    k = np.zeros((0, 1, 8), dtype=np.float32)
    with pytest.raises(ValueError, match="queries but no keys"):
        chunked_attention(q, k, k, [0, 2], [0, 0], q_chunk_tokens=2, kv_chunk_tokens=2)


def test_oracle_fully_masked_rows_are_zero_with_minus_inf_lse():
    # Bottom-right causal with more queries than keys: the first Lq - Lk rows see nothing.
    rng = np.random.default_rng(5)
    q = rng.standard_normal((6, 1, 16)).astype(np.float32)
    k = rng.standard_normal((3, 1, 16)).astype(np.float32)
    out, lse = chunked_attention(q, k, k, [0, 6], [0, 3], q_chunk_tokens=4, kv_chunk_tokens=2, causal=True)
    np.testing.assert_array_equal(out[:3], 0.0)
    assert np.all(np.isneginf(lse[:, :3]))
    assert np.all(np.isfinite(lse[:, 3:]))


def test_oracle_is_chunk_size_invariant_and_lse_identity_holds():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((50, 2, 16)).astype(np.float32)
    k = rng.standard_normal((70, 2, 16)).astype(np.float32) * 3
    v = rng.standard_normal((70, 2, 16)).astype(np.float32)
    a, la = chunked_attention(q, k, v, [0, 50], [0, 70], q_chunk_tokens=50, kv_chunk_tokens=70)
    b, lb = chunked_attention(q, k, v, [0, 50], [0, 70], q_chunk_tokens=7, kv_chunk_tokens=3)
    np.testing.assert_allclose(a, b, atol=1e-5)
    np.testing.assert_allclose(la, lb, atol=1e-5)
    # LSE == log(sum(exp(logits))) computed directly in float64
    s = np.einsum("thd,khd->htk", q.astype(np.float64), k.astype(np.float64)) * 16**-0.5
    direct = np.log(np.exp(s).sum(axis=-1))
    np.testing.assert_allclose(la, direct, atol=1e-5)


def test_oracle_row_subset_matches_full_run():
    rng = np.random.default_rng(13)
    q = rng.standard_normal((40, 3, 16)).astype(np.float32)
    k = rng.standard_normal((33, 3, 16)).astype(np.float32)
    v = rng.standard_normal((33, 3, 16)).astype(np.float32)
    rows = np.array([0, 5, 17, 39])
    full_o, full_l = chunked_attention(q, k, v, [0, 40], [0, 33], q_chunk_tokens=16, kv_chunk_tokens=8, causal=True)
    sub_o, sub_l = chunked_attention(q, k, v, [0, 40], [0, 33], q_chunk_tokens=16, kv_chunk_tokens=8,
                                     causal=True, rows=rows)
    # identical recurrence; only BLAS blocking of the smaller matmul differs
    np.testing.assert_allclose(sub_o[rows], full_o[rows], atol=1e-6)
    np.testing.assert_allclose(sub_l[:, rows], full_l[:, rows], atol=1e-6)
    assert np.isnan(sub_o[1]).all()


def test_oracle_catches_planted_mistakes():
    """A plausible bug in the recurrence must fail the closed-form check."""
    rng = np.random.default_rng(17)
    q = rng.standard_normal((12, 2, 16)).astype(np.float32)
    k = rng.standard_normal((20, 2, 16)).astype(np.float32) * 2
    v = rng.standard_normal((20, 2, 16)).astype(np.float32)
    ref_o, _ = dense_attention_f64(q, k, v, [0, 12], [0, 20])
    good, _ = chunked_attention(q, k, v, [0, 12], [0, 20], q_chunk_tokens=5, kv_chunk_tokens=6)
    assert np.abs(good - ref_o).max() < 1e-5
    # drop the alpha rescale of the accumulator (a classic online-softmax bug)
    m = np.full((2, 12), -np.inf)
    l = np.zeros((2, 12))
    o = np.zeros((2, 12, 16))
    qt = q.transpose(1, 0, 2)
    for s0 in range(0, 20, 6):
        kt = k[s0:s0 + 6].transpose(1, 0, 2)
        vt = v[s0:s0 + 6].transpose(1, 0, 2)
        s = qt @ kt.transpose(0, 2, 1) * 16**-0.5
        mm = np.maximum(m, s.max(-1))
        alpha = np.exp(m - mm)
        p = np.exp(s - mm[..., None])
        l = l * alpha + p.sum(-1)
        o = o + p @ vt  # missing "* alpha"
        m = mm
    buggy = (o / l[..., None]).transpose(1, 0, 2)
    assert np.abs(buggy - ref_o).max() > 1e-2


class _NumpyWith:
    """numpy with some functions replaced (plants a mistake in the oracle)."""

    def __init__(self, **overrides):
        self._overrides = overrides

    def __getattr__(self, name):
        return self._overrides.get(name, getattr(np, name))


def _shifted_attend(delta_shift=0, delta_pos=0):
    import oracle.seqattn_oracle as mod

    original = mod._attend_heads

    def attend(q_tile, k, v, kv_range, group, k_start, k_stop, kv_chunk, scale, causal, q_pos, shift):
        return original(q_tile, k, v, kv_range, group, k_start, k_stop, kv_chunk, scale, causal,
                        q_pos + delta_pos, shift + delta_shift)

    return attend


MUTANTS = {
    # GQA: query head h must read K/V head h // group, not h % kv_heads.
    "gqa_head_map": ("np", _NumpyWith(repeat=lambda a, r, axis: np.tile(a, (1, r, 1)))),
    # base-2 exponent where the reference's FP32 path uses natural exp
    "exp_base": ("np", _NumpyWith(exp=lambda x, out=None: np.exp2(x, out=out))),
    # bottom-right causal alignment dropped (shift Lk - Lq treated as 0)
    "causal_shift": ("_attend_heads", _shifted_attend(delta_shift=-3)),
    # query positions off by one
    "query_position": ("_attend_heads", _shifted_attend(delta_pos=1)),
}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_dense_pin_catches_mistakes_planted_in_the_oracle(mutant, monkeypatch):
    """Each plausible mistake, planted in the oracle itself, fails the dense
    float64 closed form on a causal GQA case where it matters."""
    import oracle.seqattn_oracle as mod

    rng = np.random.default_rng(23)
    q = rng.standard_normal((14, 4, 16)).astype(np.float32)
    k = rng.standard_normal((17, 2, 16)).astype(np.float32)
    v = rng.standard_normal((17, 2, 16)).astype(np.float32)
    cu_q, cu_k = [0, 14], [0, 17]
    ref_o, ref_l = dense_attention_f64(q, k, v, cu_q, cu_k, causal=True)
    good_o, good_l = chunked_attention(q, k, v, cu_q, cu_k, q_chunk_tokens=5, kv_chunk_tokens=4, causal=True)
    assert np.abs(good_o - ref_o).max() < 1e-5
    name, replacement = MUTANTS[mutant]
    monkeypatch.setattr(mod, name, replacement)
    bad_o, bad_l = chunked_attention(q, k, v, cu_q, cu_k, q_chunk_tokens=5, kv_chunk_tokens=4, causal=True)
    finite = np.isfinite(ref_l) & np.isfinite(bad_l)
    worst = max(float(np.nan_to_num(np.abs(bad_o - ref_o), nan=1.0).max()),
                float(np.abs(bad_l[finite] - ref_l[finite]).max()) if finite.any() else 0.0,
                float((np.isfinite(ref_l) != np.isfinite(bad_l)).any()))
    assert worst > 1e-3, mutant


def test_seeded_inputs_follow_torch_generator_stream():
    a = seeded_normal_chunks(10_000, 2, 8, seed=0, tensor_index=1, chunk_tokens=4096, dtype=torch.float32)
    g = torch.Generator(device="cpu").manual_seed(0 + 1 * 1_000_003 + 2)
    expected_tail = torch.empty((10_000 - 8192, 2, 8)).normal_(generator=g)
    assert torch.equal(a[8192:], expected_tail)


def test_cpu_plumbing_4096_tokens_8_heads():
    """CPU plumbing workload: fp32 [4096, 8, 64], seed 0, q block 1024, kv chunk 512 vs dense fp64."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn((4096, 8, 64), generator=g).numpy()
    k = torch.randn((4096, 8, 64), generator=g).numpy()
    v = torch.randn((4096, 8, 64), generator=g).numpy()
    cu = np.array([0, 4096])
    out, lse = chunked_attention(q, k, v, cu, cu, q_chunk_tokens=1024, kv_chunk_tokens=512)
    assert out.shape == (4096, 8, 64) and lse.shape == (8, 4096)
    rows = np.array([0, 1024, 2048, 3072, 4095, *range(7, 4096, 97)])
    ref_o, ref_l = dense_attention_f64(q, k, v, cu, cu, rows=rows)
    np.testing.assert_allclose(out[rows], ref_o[rows], atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(lse[:, rows], ref_l[:, rows], atol=2e-5)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("workers", [3, 4])
def test_head_split_and_bf16_bit_pattern_paths_equal_the_single_threaded_float_path(causal, workers):
    # The GPU configuration tests and the bench run the oracle on bf16 bit
    # patterns (uint16 views of the pinned tensors) with the K/V heads split
    # over threads.  Both must give exactly what one thread gives on the same
    # values widened to float32: 8 query heads over 4 K/V heads (GQA), ragged
    # segments, 3 workers (uneven head groups) and 4.
    from threadpoolctl import threadpool_limits

    gen = torch.Generator().manual_seed(5)
    q = torch.randn(300, 8, 64, generator=gen).to(torch.bfloat16)
    k = torch.randn(350, 4, 64, generator=gen).to(torch.bfloat16)
    v = torch.randn(350, 4, 64, generator=gen).to(torch.bfloat16)
    cu_q, cu_k = bounds([100, 200]), bounds([150, 200])

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16)

    with threadpool_limits(1):
        ref_o, ref_l = chunked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                         q_chunk_tokens=64, kv_chunk_tokens=48, causal=causal, workers=1)
        got_o, got_l = chunked_attention(bits(q), bits(k), bits(v), cu_q, cu_k, q_chunk_tokens=64,
                                         kv_chunk_tokens=48, causal=causal, workers=workers)
    assert np.isfinite(ref_o).all()
    assert np.array_equal(got_o, ref_o)
    assert np.array_equal(got_l, ref_l)
    # and the float path is itself pinned to the float64 closed form
    dense_o, dense_l = dense_attention_f64(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                           causal=causal)
    np.testing.assert_allclose(got_o, dense_o, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(got_l, dense_l, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_batch", [None, 3])
def test_torch_cpu_restatement_matches_the_oracle(causal, head_batch):
    # The CPU baseline times oracle/seqattn_torch_cpu.py; it must compute what
    # the numpy oracle computes (to float32 rounding): GQA with 8 query heads
    # over 2 K/V heads, an empty query segment, ragged chunks, more queries
    # than keys in the last segment (fully masked causal rows), bf16 inputs.
    from oracle.seqattn_torch_cpu import chunked_attention_torch

    gen = torch.Generator().manual_seed(11)
    q = torch.randn(330, 8, 64, generator=gen).to(torch.bfloat16)
    k = torch.randn(300, 2, 64, generator=gen).to(torch.bfloat16)
    v = torch.randn(300, 2, 64, generator=gen).to(torch.bfloat16)
    cu_q, cu_k = bounds([120, 0, 210]), bounds([200, 20, 80])
    ref_o, ref_l = chunked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q, cu_k,
                                     q_chunk_tokens=64, kv_chunk_tokens=48, causal=causal)
    got_o, got_l = chunked_attention_torch(q, k, v, cu_q, cu_k, q_chunk_tokens=64, kv_chunk_tokens=48,
                                           causal=causal, head_batch=head_batch)
    np.testing.assert_allclose(got_o.numpy(), ref_o, atol=2e-6, rtol=1e-5)
    ref_inf = np.isneginf(ref_l)
    assert np.array_equal(np.isneginf(got_l.numpy()), ref_inf)
    assert ref_inf.any() == causal
    np.testing.assert_allclose(got_l.numpy()[~ref_inf], ref_l[~ref_inf], atol=2e-6, rtol=1e-6)


def test_torch_cpu_restatement_pin_catches_a_planted_mistake(monkeypatch):
    # A scale dropped from the logits (a plausible slip) must fail the pin.
    import oracle.seqattn_torch_cpu as torch_cpu

    gen = torch.Generator().manual_seed(12)
    q, k, v = (torch.randn(96, 2, 32, generator=gen) for _ in range(3))
    ref_o, _ = chunked_attention(q.numpy(), k.numpy(), v.numpy(), [0, 96], [0, 96], q_chunk_tokens=32,
                                 kv_chunk_tokens=40)
    got_o, _ = torch_cpu.chunked_attention_torch(q, k, v, [0, 96], [0, 96], q_chunk_tokens=32,
                                                 kv_chunk_tokens=40, softmax_scale=1.0)
    assert np.abs(got_o.numpy() - ref_o).max() > 1e-2
